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
// Latency structure. Every thread first loads its outputs' residual (ADD
// epilogue only) and its share of x, then issues the scale loads and the
// weight loads of up to W steps, all with in-bounds clamped indices. It
// waits only for the x loads (the oldest: vmcnt counts down in issue order)
// to store x in LDS, meets the other waves at one barrier, and then consumes
// step t as soon as its own weights have arrived, while the later steps are
// still in flight. x sits in LDS transposed, [row][phase][block] (x_at), so
// a lane's S blocks of a step are one or two vector reads per row, with the
// blocks past the last full one zeroed; the tile layout holds zero codes
// there, so the padded products are fma(0, 0, acc) = acc exactly.
//
// Roofline: HBM. Bytes per call = codes + scales (+ x, out), e.g. 4,476,928 B
// for an INT8 4096x1024 matrix at one row.
#pragma once

#include "focr_internal.hpp"
#include "rms_tree.hpp"

namespace focr {
namespace gemv {

constexpr int kWaves = 4;  // waves (channel tiles) per workgroup

__device__ __forceinline__ float to_f32(int8_t v) { return static_cast<float>(static_cast<int32_t>(v)); }
__device__ __forceinline__ float to_f32(int16_t v) { return static_cast<float>(static_cast<int32_t>(v)); }
__device__ __forceinline__ float to_f32(float v) { return v; }

// Code `I` of a 16-byte weight chunk as a float, exactly (sdwa_cvt).
template <typename T, int I>
__device__ __forceinline__ float chunk_code(const uint4 &raw) {
  const uint32_t words[4] = {raw.x, raw.y, raw.z, raw.w};
  if constexpr (sizeof(T) == 1)
    return sdwa_cvt<I % 4>(words[I / 4]);
  else if constexpr (sizeof(T) == 2)
    return sdwa_cvt<4 + I % 2>(words[I / 2]);
  else
    return __uint_as_float(words[I]);
}
template <typename T, int N>
__device__ __forceinline__ void chunk_codes(const uint4 &raw, float *out) {
  if constexpr (N > 0) {
    chunk_codes<T, N - 1>(raw, out);
    out[N - 1] = chunk_code<T, N - 1>(raw);
  }
}

template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}

// Lane p < 8 of each 32-lane half: (v[p] + v[p+8]) + (v[p+16] + v[p+24]), the
// reference's (a0 + a1) + (a2 + a3) (IEEE addition is commutative, so operand
// order is immaterial). row_ror:8 pairs p with p + 8 (= p - 8 mod 16) inside a 16-lane row;
// v_permlane16_swap then pairs the two rows of each half.
__device__ __forceinline__ float fold_32_to_8(float v) {
  const float t = v + dpp<0x128>(v);
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(t), __float_as_uint(t), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Lane 0 of each half: ((v0 + v4) + (v1 + v5)) + ((v2 + v6) + (v3 + v7)):
// row_ror:12 (lane i reads lane i + 4 of its row; row_ror:n reads lane
// i - n), then quad_perm [1,0,3,2], then quad_perm [2,3,0,1].
__device__ __forceinline__ float fold_8_to_1(float v) {
  const float u = v + dpp<0x12C>(v);
  const float w = u + dpp<0xB1>(u);
  return w + dpp<0x4E>(w);
}

// One step's scales for this lane's two channels (2 * SPS floats, identical
// across the 32 lanes of a half).
template <int NS>
struct Scales {
  float v[NS > 0 ? NS : 1];
};
template <int NS>
constexpr int scale_loads() {
  return NS >= 4 ? NS / 4 : (NS == 2 ? 1 : 0);
}
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
  const float *row_scale;  // optional [rows]: x rows enter as fl(x * row_scale)
  int n, k, group, groups, nb, steps, tiles_total, glu, add;
  float *out;
};

// x in LDS, transposed: row r, phase p (0..31), block b at
// r * 32 * P + p * P + b, so that the S blocks a lane reads in one step are
// consecutive (one or two 16-byte reads instead of S 4-byte ones). P holds
// every block a step can touch, rounded to a multiple of 4 with P / 4 odd:
// the 16 lanes a ds_read_b128 serves at once then start on distinct 16-byte
// bank groups.
__host__ __device__ inline int x_phase_pitch(int steps, int S) {
  const int p = (S * steps + 3) / 4 * 4;
  return (p / 4) % 2 == 1 ? p : p + 4;
}
__host__ __device__ inline int x_pitch(int steps, int S) { return 32 * x_phase_pitch(steps, S); }
__device__ __forceinline__ int x_at(int pp, int i) { return (i & 31) * pp + (i >> 5); }

// T: code type; M: rows; SPS: scales per lane-channel per step (0 for FP32
// weights); W: steps held in registers; ROLL: steps > W, so the window is
// refilled as it is consumed (a separate instantiation, so that code common
// to both paths cannot be hoisted above the first step's wait). RMS: the row
// width whose rms_norm (unit weight, eps f32::EPSILON) each wave computes
// from the staged x while its weights are still arriving, then applies as
// fl(x * scale) on every read (0: none).
template <typename T, int M, int SPS, int W, bool ROLL, int RMS = 0>
__global__ __launch_bounds__(256) void kernel(Args a) {
  constexpr int B = sizeof(T);
  constexpr int S = 16 / (2 * B);  // 32-blocks per step
  constexpr int NS = 2 * SPS;      // scales per lane per step
  extern __shared__ float xs[];    // [M][32][pp] (x_pitch per row), then scales [kWaves][steps][2][NS]

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int h = lane >> 5, p = lane & 31;
  const int tile = blockIdx.x * kWaves + wave;
  const bool active = tile < a.tiles_total;
  const int my_tile = active ? tile : a.tiles_total - 1;
  const int k = a.k, nb = a.nb, steps = a.steps;
  const int pitch = x_pitch(steps, S), pp = x_phase_pitch(steps, S);
  const T *codes = static_cast<const T *>(a.codes);
  float *ss = xs + M * pitch;

  // Operands staged per workgroup: x (the 32 * nb floats of the full blocks
  // of each row) and the scales of the workgroup's tiles (contiguous in the
  // tile layout: kWaves * steps * 2 * NS floats from the first tile).
  const int cols = 32 * nb;
  const int cols4 = cols / 4;
  const bool x_vec = k % 4 == 0;
  const int sc_total4 = a.tiles_total * steps * 2 * NS / 4;
  const int sc_base4 = blockIdx.x * kWaves * steps * 2 * NS / 4;
  const int sc_count4 = kWaves * steps * 2 * NS / 4;
  // x[r][4i .. 4i + 3], every index clamped into the row (k >= 1; with
  // 16-byte rows k % 4 == 0 means k >= 4 whenever a float4 is read).
  // rms_norm folded in: every x element used below is fl(x * row_scale[r])
  // (rms_norm_row's `*y = *x * scale`, src/kernels/mod.rs:509-512).
  auto x_load = [&](int r, int i) {
    const float *row = a.x + static_cast<size_t>(r) * k;
    float4 v;
    if (x_vec) {
      v = reinterpret_cast<const float4 *>(row)[i * 4 + 3 < k ? i : 0];
    } else {
      auto at = [&](int c) { return row[c < k ? c : k - 1]; };
      v = make_float4(at(4 * i), at(4 * i + 1), at(4 * i + 2), at(4 * i + 3));
    }
    if (a.row_scale) {
      const float rs = a.row_scale[r];
      v = make_float4(v.x * rs, v.y * rs, v.z * rs, v.w * rs);
    }
    return v;
  };
  auto sc_load = [&](int i) {
    const int g = sc_base4 + i;
    return reinterpret_cast<const float4 *>(a.tile_scales)[g < sc_total4 ? g : sc_total4 - 1];
  };

  // 0. The ADD epilogue's residual (h), loaded first: the x loads below are
  // waited for anyway, and vmcnt counts down in issue order, so the residual
  // arrives within that wait instead of after the reduction; and the later
  // waits count only loads issued after x, so they are the same whether or
  // not this branch ran.
  const int ch0 = my_tile * kGemvChannels + h * 2;
  float res[2][M];
  if (a.add) {
#pragma unroll
    for (int c = 0; c < 2; c++)
#pragma unroll
      for (int r = 0; r < M; r++) res[c][r] = a.out[static_cast<size_t>(r) * a.n + (ch0 + c < a.n ? ch0 + c : a.n - 1)];
  } else {
#pragma unroll
    for (int c = 0; c < 2; c++)
#pragma unroll
      for (int r = 0; r < M; r++) res[c][r] = 0.0f;
  }
  __builtin_amdgcn_sched_barrier(0);

  // 1. Without ROLL: x and scales go to registers first (clamped, in bounds)
  // and to LDS only after the weight loads are issued, so their stores wait
  // for the x and scale loads only (the oldest: vmcnt counts down in issue
  // order). (The LDS-DMA path would save the registers, but a read of
  // DMA-written LDS makes the compiler wait for every load in flight.)
  constexpr int XJ = ROLL ? 1 : (8 * S * W + 255) / 256;       // float4 per thread per row
  constexpr int SJ = ROLL || NS == 0 ? 1 : (2 * W * NS + 255) / 256;  // float4 per thread
  float4 xv[M][XJ], sv[SJ];
  if constexpr (!ROLL) {
#pragma unroll
    for (int r = 0; r < M; r++)
#pragma unroll
      for (int j = 0; j < XJ; j++) {
        const int i = tid + 256 * j;
        xv[r][j] = x_load(r, i < cols4 ? i : (cols4 > 0 ? cols4 - 1 : 0));  // cols4 = 0 when k < 32
      }
    if constexpr (NS > 0)
#pragma unroll
      for (int j = 0; j < SJ; j++) sv[j] = sc_load(tid + 256 * j < sc_count4 ? tid + 256 * j : sc_count4 - 1);
  } else {
    // Rows longer than the window: stage directly (the weights wait).
    for (int r = 0; r < M; r++)
      for (int i = tid; i < cols4; i += 256) {
        const float4 v = x_load(r, i);
        float *row = xs + r * pitch;
        row[x_at(pp, 4 * i)] = v.x;
        row[x_at(pp, 4 * i + 1)] = v.y;
        row[x_at(pp, 4 * i + 2)] = v.z;
        row[x_at(pp, 4 * i + 3)] = v.w;
      }
    if constexpr (NS > 0)
      for (int i = tid; i < sc_count4; i += 256) reinterpret_cast<float4 *>(ss)[i] = sc_load(i);
  }
  __builtin_amdgcn_sched_barrier(0);

  // 2. Weights of the first W steps (clamped, in bounds).
  const uint4 *src = a.tiles + static_cast<size_t>(my_tile) * steps * 64 + lane;
  uint4 cbuf[W];
#pragma unroll
  for (int j = 0; j < W; j++) cbuf[j] = src[static_cast<size_t>(j < steps ? j : steps - 1) * 64];
  __builtin_amdgcn_sched_barrier(0);

  // 3. Store x and the scales, zero the padded blocks, and meet the other
  // waves (a plain s_barrier: __syncthreads' release fence would also wait
  // for the weight loads).
  if constexpr (!ROLL) {
#pragma unroll
    for (int r = 0; r < M; r++)
#pragma unroll
      for (int j = 0; j < XJ; j++) {
        const int i = tid + 256 * j;
        if (i < cols4) {
          float *row = xs + r * pitch;
          row[x_at(pp, 4 * i)] = xv[r][j].x;
          row[x_at(pp, 4 * i + 1)] = xv[r][j].y;
          row[x_at(pp, 4 * i + 2)] = xv[r][j].z;
          row[x_at(pp, 4 * i + 3)] = xv[r][j].w;
        }
      }
    if constexpr (NS > 0)
#pragma unroll
      for (int j = 0; j < SJ; j++)
        if (tid + 256 * j < sc_count4) reinterpret_cast<float4 *>(ss)[tid + 256 * j] = sv[j];
  }
  // Blocks nb .. pp - 1 of every phase row: zero (the padded blocks a step
  // reads past the last full one, and the pitch padding).
  for (int i = tid; i < M * 32 * (pp - nb); i += 64 * kWaves) {
    const int r = i / (32 * (pp - nb)), rest = i % (32 * (pp - nb));
    xs[r * pitch + (rest / (pp - nb)) * pp + nb + rest % (pp - nb)] = 0.0f;
  }
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  if (!active) return;
  float rsc[M];
#pragma unroll
  for (int r = 0; r < M; r++) {
    if constexpr (RMS > 0)
      rsc[r] = rms_scale_wave<RMS>([&](int i) { return xs[r * pitch + x_at(pp, i)]; }, 1.1920929e-7f);
    else
      rsc[r] = 1.0f;
  }
  const float *my_scales = ss + (wave * steps * 2 + h) * NS;  // + t * 2 * NS for step t

  float acc[2][M];
#pragma unroll
  for (int c = 0; c < 2; c++)
#pragma unroll
    for (int r = 0; r < M; r++) acc[c][r] = 0.0f;

  // Step t: S blocks of this lane's phase for both channels.
  auto step = [&](int t, const uint4 &raw) {
    float vals[S * 2];  // [block][channel], as laid out in the chunk
    chunk_codes<T, S * 2>(raw, vals);
    Scales<NS> sc;
    if constexpr (NS > 0) sc = load_scales<NS>(my_scales + t * 2 * NS);
    // This lane's S blocks of the step, for every row: consecutive in LDS.
    float xb[M][S];
#pragma unroll
    for (int r = 0; r < M; r++) {
      const float *src = xs + r * pitch + p * pp + t * S;
      if constexpr (S % 4 == 0) {
#pragma unroll
        for (int q = 0; q < S / 4; q++) {
          const float4 v = reinterpret_cast<const float4 *>(src)[q];
          xb[r][4 * q] = v.x;
          xb[r][4 * q + 1] = v.y;
          xb[r][4 * q + 2] = v.z;
          xb[r][4 * q + 3] = v.w;
        }
      } else {
        const float2 v = *reinterpret_cast<const float2 *>(src);
        xb[r][0] = v.x;
        xb[r][1] = v.y;
      }
    }
#pragma unroll
    for (int s = 0; s < S; s++) {
      float xr[M];
#pragma unroll
      for (int r = 0; r < M; r++) {
        xr[r] = xb[r][s];
        if constexpr (RMS > 0) xr[r] = xr[r] * rsc[r];
      }
#pragma unroll
      for (int c = 0; c < 2; c++) {
        float w = vals[2 * s + c];
        if constexpr (SPS > 0) w = w * sc.v[c * SPS + s / (S / SPS)];
#pragma unroll
        for (int r = 0; r < M; r++) acc[c][r] = fmaf_(xr[r], w, acc[c][r]);
      }
    }
  };
  if constexpr (!ROLL) {
#pragma unroll
    for (int t = 0; t < W; t++)
      if (t < steps) step(t, cbuf[t]);
  } else {
    for (int base = 0; base < steps; base += W) {
#pragma unroll
      for (int j = 0; j < W; j++) {
        const int t = base + j;
        if (t < steps) step(t, cbuf[j]);
        const int tn = t + W < steps ? t + W : steps - 1;
        cbuf[j] = src[static_cast<size_t>(tn) * 64];
      }
    }
  }

  auto x_col = [&](int r, int i) {
    const float v = a.x[static_cast<size_t>(r) * k + i];
    if constexpr (RMS > 0) return v * rsc[r];
    return a.row_scale ? v * a.row_scale[r] : v;
  };
#pragma unroll
  for (int c = 0; c < 2; c++)
#pragma unroll
    for (int r = 0; r < M; r++) acc[c][r] = fold_32_to_8(acc[c][r]);

  // 8-wide tail (k % 32 >= 8): one more FMA per combined lane and chunk.
  const int tail8 = (k - cols) / 8;
  for (int ci = 0; ci < tail8; ci++) {
    const int i = cols + 8 * ci;
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
#pragma unroll
  for (int c = 0; c < 2; c++)
#pragma unroll
    for (int r = 0; r < M; r++) acc[c][r] = fold_8_to_1(acc[c][r]);

  if (p != 0) return;
  float total[2][M];
#pragma unroll
  for (int c = 0; c < 2; c++) {
    const int ch = ch0 + c;
#pragma unroll
    for (int r = 0; r < M; r++) total[c][r] = acc[c][r];
    if (ch >= a.n) continue;
    // Scalar tail: total += x * fl(code * scale), unfused.
    for (int i = cols + 8 * tail8; i < k; i++) {
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
  } else if (a.add) {
    // add_residual (src/model/rope.rs:155-169): h += projected.
#pragma unroll
    for (int c = 0; c < 2; c++)
      if (ch0 + c < a.n)
#pragma unroll
        for (int r = 0; r < M; r++) {
          a.out[static_cast<size_t>(r) * a.n + ch0 + c] = res[c][r] + total[c][r];
        }
  } else {
#pragma unroll
    for (int c = 0; c < 2; c++)
      if (ch0 + c < a.n)
#pragma unroll
        for (int r = 0; r < M; r++) a.out[static_cast<size_t>(r) * a.n + ch0 + c] = total[c][r];
  }
}

// LDS bytes of one row of x, and of the workgroup's scales.
inline size_t x_row_bytes(const Linear *lin) {
  const int S = 16 / (2 * (lin->bits / 8));
  return static_cast<size_t>(x_pitch(static_cast<int>(lin->gemv_steps), S)) * sizeof(float);
}
inline size_t scale_lds_bytes(const Linear *lin) { return kWaves * lin->gemv_steps * 2 * 2 * lin->gemv_sps * sizeof(float); }
constexpr size_t kLdsBudget = 64 * 1024;

template <typename T, int M, int SPS, int W, bool ROLL = false, int RMS = 0>
int launch_typed(Ctx *ctx, const Linear *lin, const float *x, const float *rs, float *out, int epi) {
  const size_t lds = M * x_row_bytes(lin) + scale_lds_bytes(lin);
  FOCR_REQUIRE(lds <= kLdsBudget, FOCR_E_SHAPE, "GEMV: x rows exceed the LDS budget");
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
  a.row_scale = rs;
  a.n = static_cast<int>(lin->n);
  a.k = static_cast<int>(lin->k);
  a.group = static_cast<int>(lin->group);
  a.groups = static_cast<int>(lin->groups);
  a.nb = static_cast<int>(lin->gemv_blocks);
  a.steps = static_cast<int>(lin->gemv_steps);
  a.tiles_total = static_cast<int>(lin->gemv_tiles);
  a.glu = epi == FOCR_EPI_GLU ? 1 : 0;
  a.add = epi == FOCR_EPI_ADD ? 1 : 0;
  a.out = out;
  hipLaunchKernelGGL((kernel<T, M, SPS, W, ROLL, RMS>), dim3(blocks), dim3(64 * kWaves), lds, ctx->stream, a);
  FOCR_HIP_CHECK(hipGetLastError());
  return FOCR_OK;
}

// The in-kernel rms_norm is instantiated for the model's hidden width.
constexpr int kRmsWidth = 768;

// Window buckets: every step in registers up to 20 steps (FP32: 36), which
// covers every matrix of the model; longer rows refill a 20 (36) step window.
// rs == kRmsInKernel selects the in-kernel rms_norm (in_dim == kRmsWidth).
template <typename T, int M, int SPS>
int launch_window(Ctx *ctx, const Linear *lin, const float *x, const float *rs, float *out, int epi) {
  const size_t steps = lin->gemv_steps;
  if (rs == kRmsInKernel) {
    constexpr int B = sizeof(T), S = 16 / (2 * B);
    constexpr int RW = (kRmsWidth / 32 + S - 1) / S;  // steps of a kRmsWidth row
    constexpr int WB = RW <= 4 ? 4 : RW <= 8 ? 8 : RW <= 12 ? 12 : 20;
    return launch_typed<T, M, SPS, WB, false, kRmsWidth>(ctx, lin, x, nullptr, out, epi);
  }
  if (steps <= 4) return launch_typed<T, M, SPS, 4>(ctx, lin, x, rs, out, epi);
  if (steps <= 8) return launch_typed<T, M, SPS, 8>(ctx, lin, x, rs, out, epi);
  if (steps <= 12) return launch_typed<T, M, SPS, 12>(ctx, lin, x, rs, out, epi);
  if (steps <= 20) return launch_typed<T, M, SPS, 20>(ctx, lin, x, rs, out, epi);
  if constexpr (SPS == 0) {
    if (steps <= 36) return launch_typed<T, M, SPS, 36>(ctx, lin, x, rs, out, epi);
    return launch_typed<T, M, SPS, 36, true>(ctx, lin, x, rs, out, epi);
  } else {
    return launch_typed<T, M, SPS, 20, true>(ctx, lin, x, rs, out, epi);
  }
}

template <typename T, int SPS>
int launch_rows(Ctx *ctx, const Linear *lin, const float *x, const float *rs, size_t rows, float *out, int epi) {
  switch (rows) {
    case 1: return launch_window<T, 1, SPS>(ctx, lin, x, rs, out, epi);
    case 2: return launch_window<T, 2, SPS>(ctx, lin, x, rs, out, epi);
    case 3: return launch_window<T, 3, SPS>(ctx, lin, x, rs, out, epi);
    case 4: return launch_window<T, 4, SPS>(ctx, lin, x, rs, out, epi);
    case 5: return launch_window<T, 5, SPS>(ctx, lin, x, rs, out, epi);
    case 6: return launch_window<T, 6, SPS>(ctx, lin, x, rs, out, epi);
    case 7: return launch_window<T, 7, SPS>(ctx, lin, x, rs, out, epi);
    case 8: return launch_window<T, 8, SPS>(ctx, lin, x, rs, out, epi);
    default: return set_error(FOCR_E_SHAPE, "GEMV rows must be 1..=8");
  }
}

// Per-code-type dispatch (one translation unit each, compiled in parallel).
int launch_i8(Ctx *ctx, const Linear *lin, const float *x, const float *rs, size_t rows, float *out, int epi);
int launch_i16(Ctx *ctx, const Linear *lin, const float *x, const float *rs, size_t rows, float *out, int epi);
int launch_f32(Ctx *ctx, const Linear *lin, const float *x, const float *rs, size_t rows, float *out, int epi);

}  // namespace gemv
}  // namespace focr
