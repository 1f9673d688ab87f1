// Fast-mode prefill projection: INT16 activations x INT8 weight codes, the
// reference's INT16 panels (src/kernels/panels/panel_i16.rs), bitwise.
//
// 1. quantize_kernel: every 64-input group of every row becomes INT16 codes
//    q and a step (quantize_group, panel_i16.rs:233-266; pack_rows 275-329:
//    exception columns zeroed first, step times the row scale, exception
//    inputs x * row_scale kept in FP32). Each code is split exactly as
//    q = 256*h + (l + 128) with h, l in [-128, 127], and h and l are written
//    as two int8 planes in the lane order of the 16x16x64 i8 matrix-core
//    operand, so every wave load in the GEMM is one contiguous 1 KB chunk.
// 2. gemm_kernel: per 16x16 output block and group, two i8 MFMAs give the
//    group's exact INT32 sum: H = sum h*w; C = (H << 8) + 128*sum(w) (the last
//    term precomputed per column at upload); S = C + sum l*w. |S| < 2^31 as
//    in the reference (64 * 32767 * 127). Then, in the reference's order,
//    acc = fma(f32(S), fl(s_w * s_a), acc) over ascending groups, the
//    exception FMAs ascending, and the epilogue (Store, Glu, Add).
// Because the group sums are exact integers, any summation order inside the
// matrix core gives the same S, and every output matches kernel_scalar bit
// for bit.
//
// Each group's A and B tiles, activation steps, column sums and scales are
// copied HBM -> LDS by the LDS-DMA path into one of two buffers while the
// previous group is computed from the other.
//
// Roofline: the i8 matrix cores do 2 x 64 MACs per output and group; the
// FP32 group epilogue (4 VALU ops per output and group) bounds it in practice.
#include "focr_internal.hpp"

namespace focr {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int kBM = 128;  // rows per workgroup tile
constexpr int kBN = 128;  // columns per workgroup tile

// One wave per (16-row block, group): lane l owns row l%16, inputs
// 16*(l/16) .. +16 of the group; the group's absmax is a 4-lane reduction.
__global__ __launch_bounds__(256) void quantize_kernel(const float *__restrict__ x, int m, int k, int groups,
                                                       int row_blocks, const float *__restrict__ row_scale,
                                                       const int16_t *__restrict__ exc_index, int n_exc,
                                                       int8_t *__restrict__ a_tiles, float *__restrict__ steps,
                                                       float *__restrict__ exc_inputs, int m_pad) {
  const int wave = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (wave >= row_blocks * groups) return;
  const int g = wave / row_blocks, mb = wave % row_blocks;
  const int lane = threadIdx.x & 63;
  const int row = mb * 16 + (lane & 15);
  const int k0 = g * 64 + 16 * (lane >> 4);
  float v[16];
  const bool live = row < m;
  if (live) {
    const float4 *src = reinterpret_cast<const float4 *>(x + static_cast<size_t>(row) * k + k0);
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const float4 f = src[i];
      v[4 * i] = f.x;
      v[4 * i + 1] = f.y;
      v[4 * i + 2] = f.z;
      v[4 * i + 3] = f.w;
    }
  } else {
#pragma unroll
    for (int i = 0; i < 16; i++) v[i] = 0.0f;
  }
  const float scale = live ? (row_scale ? row_scale[row] : 1.0f) : 0.0f;
  // Exception columns: keep x * row_scale, quantize the group without them.
  if (exc_index) {
#pragma unroll
    for (int i = 0; i < 16; i++) {
      const int e = exc_index[k0 + i];
      if (e >= 0) {
        if (live) exc_inputs[static_cast<size_t>(row) * n_exc + e] = v[i] * scale;
        v[i] = 0.0f;
      }
    }
  }
  // absmax from bit patterns (NaN and infinity order above every finite value).
  uint32_t top = 0;
#pragma unroll
  for (int i = 0; i < 16; i++) {
    const uint32_t b = __float_as_uint(v[i]) & 0x7fffffffu;
    top = b > top ? b : top;
  }
  {
    uint32_t o = static_cast<uint32_t>(__shfl_xor(static_cast<int>(top), 16));
    top = o > top ? o : top;
    o = static_cast<uint32_t>(__shfl_xor(static_cast<int>(top), 32));
    top = o > top ? o : top;
  }
  int q[16];
  float step;
  const float qmax = 32767.0f;
  if (top >= 0x7f800000u) {
#pragma unroll
    for (int i = 0; i < 16; i++) q[i] = 0;
    step = __builtin_nanf("");
  } else {
    const float absmax = __uint_as_float(top);
    const float inv = __fdiv_rn(qmax, absmax);
    if (!__builtin_isfinite(inv)) {
      if (absmax == 0.0f) {
#pragma unroll
        for (int i = 0; i < 16; i++) q[i] = 0;
        step = 0.0f;
      } else {
        // The reciprocal overflows: an f64 path with the step rounded up
        // where its rounding would clip the maximum.
        step = __fdiv_rn(absmax, qmax);
        const float tiny = __uint_as_float(1u);
        step = step > tiny ? step : tiny;
        if (static_cast<double>(step) * 32767.0 < static_cast<double>(absmax))
          step = __uint_as_float(__float_as_uint(step) + 1u);
#pragma unroll
        for (int i = 0; i < 16; i++) {
          double r = __builtin_rint(__ddiv_rn(static_cast<double>(v[i]), static_cast<double>(step)));
          r = r < -32767.0 ? -32767.0 : (r > 32767.0 ? 32767.0 : r);
          q[i] = static_cast<int>(r);
        }
      }
    } else {
      const float magic = 12582912.0f;  // 1.5 * 2^23
#pragma unroll
      for (int i = 0; i < 16; i++) {
        float y = v[i] * inv;
        y = y < -qmax ? -qmax : (y > qmax ? qmax : y);
        q[i] = static_cast<int>(__float_as_uint(y + magic)) - static_cast<int>(__float_as_uint(magic));
      }
      step = __fdiv_rn(absmax, qmax);
    }
  }
  // q = 256 * h + (l + 128), h = q >> 8, l = (q & 255) - 128.
  uint32_t hi[4], lo[4];
#pragma unroll
  for (int w = 0; w < 4; w++) {
    uint32_t hw = 0, lw = 0;
#pragma unroll
    for (int b = 0; b < 4; b++) {
      const int c = q[4 * w + b];
      hw |= (static_cast<uint32_t>(c >> 8) & 0xffu) << (8 * b);
      lw |= (static_cast<uint32_t>((c & 0xff) - 128) & 0xffu) << (8 * b);
    }
    hi[w] = hw;
    lo[w] = lw;
  }
  int8_t *dst = a_tiles + (static_cast<size_t>(g) * row_blocks + mb) * 2048;
  reinterpret_cast<uint4 *>(dst)[lane] = make_uint4(hi[0], hi[1], hi[2], hi[3]);
  reinterpret_cast<uint4 *>(dst + 1024)[lane] = make_uint4(lo[0], lo[1], lo[2], lo[3]);
  if (lane < 16) steps[static_cast<size_t>(g) * m_pad + row] = step * scale;
}

// One group's operands in LDS, filled by the LDS-DMA path (25.5 KB; two
// buffers).
struct GroupTile {
  uint4 a[kBM / 16 * 2 * 64];  // [8 row blocks][hi, lo][64 lanes] x 16 B
  uint4 b[kBN / 16 * 64];      // [8 column blocks][64 lanes] x 16 B
  float steps[kBM];            // activation steps of the tile's rows
  int32_t wsum[kBN];           // 128 * sum of the group's codes per column
  float sw[kBN];               // weight scales per column
};

typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(1))) const void global_void;

// NB: 16-column blocks per wave (4: 128-column workgroup tiles; 2: 64-column
// tiles, the ones launched).
template <int EPI, int NB>
__global__ __launch_bounds__(256) void gemm_kernel(const int8_t *__restrict__ a_tiles, const float *__restrict__ steps,
                                                   const float *__restrict__ exc_inputs, const int8_t *__restrict__ b_tiles,
                                                   const int32_t *__restrict__ wsum, const float *__restrict__ sw,
                                                   const float *__restrict__ exc_vals, int n_exc, int m, int n,
                                                   int groups, int row_blocks, int m_pad, float *__restrict__ out) {
  __shared__ GroupTile buf0;
  __shared__ GroupTile buf1;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  const int mb0 = blockIdx.x * (kBM / 16);
  const int nb0 = blockIdx.y * (2 * NB);
  const int col_blocks = n / 16;

  // Group g -> t by DMA (16 B per lane; sources clamped into their arrays,
  // columns past n are computed and discarded): A 4 and B 2 instructions per
  // thread; the steps, column sums and scales by lanes 0-31 of waves 0-2.
  auto copy_group = [&](GroupTile &t, int g) {
    const char *ga = reinterpret_cast<const char *>(a_tiles) + (static_cast<size_t>(g) * row_blocks + mb0) * 2048;
#pragma unroll
    for (int i = 0; i < 4; i++)
      __builtin_amdgcn_global_load_lds((global_void *)(ga + 16 * (tid + 256 * i)), (lds_void *)(&t.a[64 * wave + 256 * i]),
                                       16, 0, 0);
#pragma unroll
    for (int i = 0; i < NB / 2; i++) {
      const int idx = tid + 256 * i;
      int blk = nb0 + idx / 64;
      blk = blk < col_blocks ? blk : col_blocks - 1;
      const char *gb = reinterpret_cast<const char *>(b_tiles) + ((static_cast<size_t>(g) * col_blocks + blk) * 64 + (idx & 63)) * 16;
      __builtin_amdgcn_global_load_lds((global_void *)gb, (lds_void *)(&t.b[64 * wave + 256 * i]), 16, 0, 0);
    }
    if (lane < 32) {
      if (wave == 0) {
        __builtin_amdgcn_global_load_lds((global_void *)(steps + static_cast<size_t>(g) * m_pad + mb0 * 16 + 4 * lane),
                                         (lds_void *)(&t.steps[0]), 16, 0, 0);
      } else if (wave < 3) {
        int col = nb0 * 16 + 4 * lane;
        col = col < n ? col : n - 4;
        const void *src = wave == 1 ? static_cast<const void *>(wsum + static_cast<size_t>(g) * n + col)
                                    : static_cast<const void *>(sw + static_cast<size_t>(g) * n + col);
        __builtin_amdgcn_global_load_lds((global_void *)src, wave == 1 ? (lds_void *)(&t.wsum[0]) : (lds_void *)(&t.sw[0]),
                                         16, 0, 0);
      }
    }
  };

  float acc[4][NB][4];
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int j = 0; j < NB; j++)
#pragma unroll
      for (int r = 0; r < 4; r++) acc[i][j][r] = 0.0f;

  const int quad = lane >> 4, col_in = lane & 15;
  // Group g is read from one buffer while g + 1 is copied into the other.
  auto step = [&](GroupTile &cur, GroupTile &next, int g) __attribute__((always_inline)) {
    __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0): this wave's copies of cur
    __syncthreads();                     // everyone's; nobody still reads next
    if (g + 1 < groups) copy_group(next, g + 1);
    v4i ahi[4], alo[4], b[NB];
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int rb = wm * 4 + i;
      const uint4 hv = cur.a[(rb * 2) * 64 + lane], lv = cur.a[(rb * 2 + 1) * 64 + lane];
      ahi[i] = v4i{static_cast<int>(hv.x), static_cast<int>(hv.y), static_cast<int>(hv.z), static_cast<int>(hv.w)};
      alo[i] = v4i{static_cast<int>(lv.x), static_cast<int>(lv.y), static_cast<int>(lv.z), static_cast<int>(lv.w)};
    }
#pragma unroll
    for (int j = 0; j < NB; j++) {
      const uint4 w = cur.b[(wn * NB + j) * 64 + lane];
      b[j] = v4i{static_cast<int>(w.x), static_cast<int>(w.y), static_cast<int>(w.z), static_cast<int>(w.w)};
    }
    int32_t ws[NB];
    float swv[NB];
#pragma unroll
    for (int j = 0; j < NB; j++) {
      const int c = (wn * NB + j) * 16 + col_in;
      ws[j] = cur.wsum[c];
      swv[j] = cur.sw[c];
    }
    float sa[4][4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const float4 sv = *reinterpret_cast<const float4 *>(&cur.steps[(wm * 4 + i) * 16 + 4 * quad]);
      sa[i][0] = sv.x;
      sa[i][1] = sv.y;
      sa[i][2] = sv.z;
      sa[i][3] = sv.w;
    }
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
      for (int j = 0; j < NB; j++) {
        const v4i zero = {0, 0, 0, 0};
        v4i hsum = __builtin_amdgcn_mfma_i32_16x16x64_i8(ahi[i], b[j], zero, 0, 0, 0);
        v4i c;
#pragma unroll
        for (int r = 0; r < 4; r++) c[r] = (hsum[r] << 8) + ws[j];
        const v4i sum = __builtin_amdgcn_mfma_i32_16x16x64_i8(alo[i], b[j], c, 0, 0, 0);
#pragma unroll
        for (int r = 0; r < 4; r++) {
          const float scale = swv[j] * sa[i][r];
          acc[i][j][r] = fmaf_(static_cast<float>(sum[r]), scale, acc[i][j][r]);
        }
      }
  };
  copy_group(buf0, 0);
  for (int g = 0; g < groups; g += 2) {
    step(buf0, buf1, g);
    if (g + 1 < groups) step(buf1, buf0, g + 1);
  }

  // Exception FMAs (ascending columns), then the epilogue.
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int row_base = (mb0 + wm * 4 + i) * 16 + 4 * quad;
#pragma unroll
    for (int j = 0; j < NB; j++) {
      const int col = (nb0 + wn * NB + j) * 16 + col_in;
      const bool col_ok = col < n;
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const int row = row_base + r;
        float v = acc[i][j][r];
        if (n_exc && col_ok && row < m)
          for (int e = 0; e < n_exc; e++)
            v = fmaf_(exc_inputs[static_cast<size_t>(row) * n_exc + e], exc_vals[static_cast<size_t>(col) * n_exc + e], v);
        if constexpr (EPI == FOCR_EPI_GLU) {
          const float up = __shfl_xor(v, 1);
          if (col_ok && row < m && (col & 1) == 0)
            out[static_cast<size_t>(row) * (n / 2) + col / 2] = squared_relu_glu(v, up);
        } else if constexpr (EPI == FOCR_EPI_ADD) {
          if (col_ok && row < m) {
            float *dst = out + static_cast<size_t>(row) * n + col;
            *dst = *dst + v;
          }
        } else {
          if (col_ok && row < m) out[static_cast<size_t>(row) * n + col] = v;
        }
      }
    }
  }
}

}  // namespace

int launch_prefill_i16(Ctx *ctx, const Linear *lin, const float *x, size_t rows, const float *row_scale,
                       int epilogue, float *out) {
  const size_t m = rows, k = lin->k, n = lin->n, groups = lin->groups;
  FOCR_REQUIRE(m < (size_t(1) << 30) && n % 32 == 0 && k % 64 == 0, FOCR_E_SHAPE, "INT16 panel shape");
  const size_t m_pad = (m + kBM - 1) / kBM * kBM;
  const size_t row_blocks = m_pad / 16;
  const size_t a_bytes = m_pad * k * 2;
  const size_t s_bytes = groups * m_pad * sizeof(float);
  const size_t e_bytes = m_pad * (lin->n_exc ? lin->n_exc : 1) * sizeof(float);
  int rc = ensure_scratch(ctx, a_bytes + s_bytes + e_bytes + 256);
  if (rc != FOCR_OK) return rc;
  int8_t *a_tiles = static_cast<int8_t *>(ctx->scratch);
  float *steps = reinterpret_cast<float *>(static_cast<char *>(ctx->scratch) + a_bytes);
  float *exc_inputs = reinterpret_cast<float *>(static_cast<char *>(ctx->scratch) + a_bytes + s_bytes);

  const size_t waves = row_blocks * groups;
  hipLaunchKernelGGL(quantize_kernel, dim3(static_cast<unsigned>((waves + 3) / 4)), dim3(256), 0, ctx->stream, x,
                     static_cast<int>(m), static_cast<int>(k), static_cast<int>(groups), static_cast<int>(row_blocks),
                     row_scale, lin->exc_index, static_cast<int>(lin->n_exc), a_tiles, steps, exc_inputs,
                     static_cast<int>(m_pad));
  FOCR_HIP_CHECK(hipGetLastError());
  // 64-column workgroup tiles (two 16-column blocks per wave): twice the
  // workgroups of 128-column tiles, measured faster on every shape (m = 6,544:
  // literal 0.130 -> 0.115 ms, W13 0.118 -> 0.106, QKV 0.062 -> 0.057,
  // WO 0.058 -> 0.046, W2 0.096 -> 0.075).
  constexpr int kNB = 2;
  const dim3 grid(static_cast<unsigned>(m_pad / kBM), static_cast<unsigned>((n + 32 * kNB - 1) / (32 * kNB)));
#define FOCR_LAUNCH_I16(E)                                                                                      \
  hipLaunchKernelGGL((gemm_kernel<E, kNB>), grid, dim3(256), 0, ctx->stream, a_tiles, steps, exc_inputs, lin->i16_b, \
                     lin->i16_wsum, lin->i16_sw, lin->exc_vals, static_cast<int>(lin->n_exc), static_cast<int>(m), \
                     static_cast<int>(n), static_cast<int>(groups), static_cast<int>(row_blocks),                \
                     static_cast<int>(m_pad), out)
  if (epilogue == FOCR_EPI_GLU)
    FOCR_LAUNCH_I16(FOCR_EPI_GLU);
  else if (epilogue == FOCR_EPI_ADD)
    FOCR_LAUNCH_I16(FOCR_EPI_ADD);
  else
    FOCR_LAUNCH_I16(FOCR_EPI_STORE);
#undef FOCR_LAUNCH_I16
  FOCR_HIP_CHECK(hipGetLastError());
  return FOCR_OK;
}

}  // namespace focr
