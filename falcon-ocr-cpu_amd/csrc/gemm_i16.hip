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

template <int EPI>
__global__ __launch_bounds__(256) void gemm_kernel(const int8_t *__restrict__ a_tiles, const float *__restrict__ steps,
                                                   const float *__restrict__ exc_inputs, const int8_t *__restrict__ b_tiles,
                                                   const int32_t *__restrict__ wsum, const float *__restrict__ sw,
                                                   const float *__restrict__ exc_vals, int n_exc, int m, int n,
                                                   int groups, int row_blocks, int m_pad, float *__restrict__ out) {
  __shared__ uint4 lds_a[kBM / 16 * 2 * 64];  // [8 row blocks][hi, lo][64 lanes] x 16 B
  __shared__ uint4 lds_b[kBN / 16 * 64];      // [8 col blocks][64 lanes] x 16 B
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int mb0 = blockIdx.x * (kBM / 16);
  const int nb0 = blockIdx.y * (kBN / 16);
  const int col_blocks = n / 16;

  float acc[4][4][4];
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int j = 0; j < 4; j++)
#pragma unroll
      for (int r = 0; r < 4; r++) acc[i][j][r] = 0.0f;

  const int quad = lane >> 4, col_in = lane & 15;
  for (int g = 0; g < groups; g++) {
    // Stage this group's operands: A 16 KB (contiguous), B up to 8 KB.
    const uint4 *ga = reinterpret_cast<const uint4 *>(a_tiles + (static_cast<size_t>(g) * row_blocks + mb0) * 2048);
#pragma unroll
    for (int i = 0; i < 4; i++) lds_a[tid + 256 * i] = ga[tid + 256 * i];
    const uint4 *gb = reinterpret_cast<const uint4 *>(b_tiles + (static_cast<size_t>(g) * col_blocks + nb0) * 1024);
#pragma unroll
    for (int i = 0; i < 2; i++) {
      const int idx = tid + 256 * i;
      if (nb0 + idx / 64 < col_blocks) lds_b[idx] = gb[idx];
    }
    __syncthreads();
    v4i ahi[4], alo[4], b[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int rb = wm * 4 + i;
      const uint4 h = lds_a[(rb * 2) * 64 + lane], l = lds_a[(rb * 2 + 1) * 64 + lane];
      ahi[i] = v4i{static_cast<int>(h.x), static_cast<int>(h.y), static_cast<int>(h.z), static_cast<int>(h.w)};
      alo[i] = v4i{static_cast<int>(l.x), static_cast<int>(l.y), static_cast<int>(l.z), static_cast<int>(l.w)};
    }
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const uint4 w = lds_b[(wn * 4 + j) * 64 + lane];
      b[j] = v4i{static_cast<int>(w.x), static_cast<int>(w.y), static_cast<int>(w.z), static_cast<int>(w.w)};
    }
    __syncthreads();
    // Per-column weight terms and per-row activation steps of this group.
    int32_t ws[4];
    float swv[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const int col = (nb0 + wn * 4 + j) * 16 + col_in;
      const int c = col < n ? col : n - 1;
      ws[j] = wsum[static_cast<size_t>(g) * n + c];
      swv[j] = sw[static_cast<size_t>(g) * n + c];
    }
    float sa[4][4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int row = (mb0 + wm * 4 + i) * 16 + 4 * quad;
      const float4 s = *reinterpret_cast<const float4 *>(steps + static_cast<size_t>(g) * m_pad + row);
      sa[i][0] = s.x;
      sa[i][1] = s.y;
      sa[i][2] = s.z;
      sa[i][3] = s.w;
    }
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const v4i zero = {0, 0, 0, 0};
        v4i hsum = __builtin_amdgcn_mfma_i32_16x16x64_i8(ahi[i], b[j], zero, 0, 0, 0);
        v4i c;
#pragma unroll
        for (int r = 0; r < 4; r++) c[r] = (hsum[r] << 8) + ws[j];
        const v4i s = __builtin_amdgcn_mfma_i32_16x16x64_i8(alo[i], b[j], c, 0, 0, 0);
#pragma unroll
        for (int r = 0; r < 4; r++) {
          const float scale = swv[j] * sa[i][r];
          acc[i][j][r] = fmaf_(static_cast<float>(s[r]), scale, acc[i][j][r]);
        }
      }
  }

  // Exception FMAs (ascending columns), then the epilogue.
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int row_base = (mb0 + wm * 4 + i) * 16 + 4 * quad;
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const int col = (nb0 + wn * 4 + j) * 16 + col_in;
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
  const dim3 grid(static_cast<unsigned>(m_pad / kBM), static_cast<unsigned>((n + kBN - 1) / kBN));
#define FOCR_LAUNCH_I16(E)                                                                                      \
  hipLaunchKernelGGL(gemm_kernel<E>, grid, dim3(256), 0, ctx->stream, a_tiles, steps, exc_inputs, lin->i16_b,   \
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
