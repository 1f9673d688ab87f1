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
// copied HBM -> LDS by the LDS-DMA path into one of two stages while the
// previous group is computed from the other; tiles are ordered per XCD so
// that the workgroups sharing an L2 share operands.
//
// Roofline: the i8 matrix cores do 2 x 64 MACs per output and group, the
// FP32 group epilogue 4 VALU ops per output and group (shift-add and convert
// issue at half the FMA rate). Measured, neither bounds it alone: without the
// epilogue it runs about 25 % faster, without the products about 15 %; the
// operand copies (L2 -> LDS, about 1 GB per 6544 x 1024 x 4096 call) and the
// per-group barrier take the rest.
#include "focr_internal.hpp"

namespace focr {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int kMPad = 128;  // rows padded to a multiple of this
constexpr int kBM = 64;     // rows per workgroup tile

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

// One group's operands of a 64 x BN tile in LDS, filled by the LDS-DMA path;
// two stages (the group being computed and the next one).
template <int BN>
struct GroupTile {
  uint4 a[kBM / 16 * 2 * 64];  // [4 row blocks][hi, lo][64 lanes] x 16 B
  uint4 b[BN / 16 * 64];       // [column blocks][64 lanes] x 16 B
  float steps[kBM];            // activation steps of the tile's rows
  int32_t wsum[BN];            // 128 * sum of the group's codes per column
  float sw[BN];                // weight scales per column
};

typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(1))) const void global_void;

// Compiler-only ordering around the plain workgroup barrier: the waits are
// explicit (a __syncthreads fence would wait for every copy in flight).
__device__ __forceinline__ void plain_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// Tile order. Workgroups are dealt to the 8 XCDs round robin (block b runs on
// XCD b % 8); block b takes tile t = (b % 8) * per + b / 8 so that each XCD
// walks one contiguous run of tiles, and tiles run in panels of kPanel row
// tiles, column tiles in order, rows fastest: the workgroups an XCD holds at
// once share a few A row tiles and B column tiles in its own L2.
constexpr int kPanel = 4;
__device__ __forceinline__ void tile_of(int b, int row_tiles, int col_tiles, int &rt, int &ct) {
  const int total = row_tiles * col_tiles;
  const int per = total / 8;
  const int t = b < 8 * per ? (b % 8) * per + b / 8 : b;
  const int panel = t / (kPanel * col_tiles);
  const int rem = t - panel * kPanel * col_tiles;
  const int rows = row_tiles - panel * kPanel < kPanel ? row_tiles - panel * kPanel : kPanel;
  ct = rem / rows;
  rt = panel * kPanel + rem % rows;
}

// 64 x BN outputs per workgroup of BN / 16 waves; wave (wm, wn) holds 32
// rows x 32 columns, 2 row blocks x 2 column blocks of 16 x 16. A wider tile
// moves fewer operand bytes per output (the activation planes are copied once
// per BN columns, the weights once per 64 rows).
//
// Step g: wait for this wave's copies of group g, meet the other waves
// (nobody still reads the other stage), start group g + 1's copies into it,
// then compute group g: per block two i8 matrix-core products and the FP32
// epilogue acc = fma(f32(S), fl(s_w * s_a), acc). 128-column tiles hold 8
// waves; at most 80 VGPRs keep three such workgroups (6 waves per SIMD) on a
// compute unit.
template <int EPI, int BN>
__global__ __launch_bounds__(BN * 4) __attribute__((amdgpu_waves_per_eu(BN == 128 ? 6 : 1)))
void gemm_kernel(const int8_t *__restrict__ a_tiles, const float *__restrict__ steps,
                                                   const float *__restrict__ exc_inputs, const int8_t *__restrict__ b_tiles,
                                                   const int32_t *__restrict__ wsum, const float *__restrict__ sw,
                                                   const float *__restrict__ exc_vals, int n_exc, int m, int n,
                                                   int groups, int row_blocks, int m_pad, int row_tiles, int col_tiles,
                                                   float *__restrict__ out) {
  constexpr int RB = kBM / 16, RW = 2, WAVES = BN / 16, THREADS = 64 * WAVES;
  constexpr int ACP = RB * 2 * 64 / THREADS;  // A copies per thread and group
  typedef GroupTile<BN> Tile;
  // Two distinct LDS objects (not one array): the compiler then sees that
  // reads of one stage do not alias copies into the other.
  __shared__ Tile ring0, ring1;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / (BN / 32), wn = wave % (BN / 32);
  int rt, ct;
  tile_of(blockIdx.x, row_tiles, col_tiles, rt, ct);
  const int mb0 = rt * RB;
  const int nb0 = ct * (BN / 16);
  const int col_blocks = n / 16;

  // Sources of this thread's copies per group, each a uniform base (scalar
  // registers, advanced by a group's stride) plus a 32-bit lane offset so that
  // every copy takes the scalar-base address form: ACP x 16 B of the A planes;
  // 16 B of column block nb0 + wave of B (blocks past n repeat the last one:
  // computed and discarded); and, for waves 0 .. 2 BN / 64, 4 B of the steps
  // (wave 0), of the column sums or of the scales (64 columns per wave).
  const char *abase = reinterpret_cast<const char *>(a_tiles) + static_cast<size_t>(mb0) * 2048;
  const uint32_t aoff = 16u * tid;
  const size_t a_stride = static_cast<size_t>(row_blocks) * 2048;
  const char *bbase = reinterpret_cast<const char *>(b_tiles) + static_cast<size_t>(nb0) * 1024;
  int blk = nb0 + wave;
  blk = blk < col_blocks ? blk : col_blocks - 1;
  const uint32_t boff = static_cast<uint32_t>((blk - nb0) * 64 + lane) * 16u;
  const size_t b_stride = static_cast<size_t>(col_blocks) * 1024;
  constexpr int XP = BN / 64;  // 64-column pieces of the sums and of the scales
  const bool x_copy = wave <= 2 * XP;
  const char *xbase = reinterpret_cast<const char *>(steps + mb0 * 16);
  uint32_t xoff = 4u * lane;
  size_t x_stride = static_cast<size_t>(m_pad) * sizeof(float);
  int x_dst = static_cast<int>(offsetof(Tile, steps));  // byte offset of the wave's 256 B in the stage
  if (wave != 0 && x_copy) {
    const bool scales = wave > XP;
    const int piece = scales ? wave - 1 - XP : wave - 1;
    int col = nb0 * 16 + 64 * piece + lane;
    col = col < n ? col : n - 1;
    xbase = scales ? reinterpret_cast<const char *>(sw + nb0 * 16) : reinterpret_cast<const char *>(wsum + nb0 * 16);
    xoff = 4u * static_cast<uint32_t>(col - nb0 * 16);
    x_stride = static_cast<size_t>(n) * 4;
    x_dst = (scales ? static_cast<int>(offsetof(Tile, sw)) : static_cast<int>(offsetof(Tile, wsum))) + 256 * piece;
  }
  auto issue = [&](Tile &t, int g) {
    const char *ga = abase + static_cast<size_t>(g) * a_stride;
#pragma unroll
    for (int i = 0; i < ACP; i++)
      __builtin_amdgcn_global_load_lds((global_void *)((ga + 16 * THREADS * i) + aoff),
                                       (lds_void *)(&t.a[64 * wave + THREADS * i]), 16, 0, 0);
    __builtin_amdgcn_global_load_lds((global_void *)(bbase + static_cast<size_t>(g) * b_stride + boff),
                                     (lds_void *)(&t.b[64 * wave]), 16, 0, 0);
    if (x_copy)
      __builtin_amdgcn_global_load_lds((global_void *)(xbase + static_cast<size_t>(g) * x_stride + xoff),
                                       (lds_void *)(reinterpret_cast<char *>(&t) + x_dst), 4, 0, 0);
  };

  float acc[RW][2][4];
#pragma unroll
  for (int i = 0; i < RW; i++)
#pragma unroll
    for (int j = 0; j < 2; j++)
#pragma unroll
      for (int r = 0; r < 4; r++) acc[i][j][r] = 0.0f;

  const int quad = lane >> 4, col_in = lane & 15;
  auto step = [&](Tile &cur, Tile &next, int g) __attribute__((always_inline)) {
    __builtin_amdgcn_s_waitcnt(0x0070);  // vmcnt(0) lgkmcnt(0): group g landed
    plain_barrier();
    // Past the last group the copy repeats it into the free stage.
    issue(next, g + 1 < groups ? g + 1 : groups - 1);
    v4i ahi[RW], alo[RW], b[2];
#pragma unroll
    for (int i = 0; i < RW; i++) {
      const int rb = wm * RW + i;
      const uint4 hv = cur.a[(rb * 2) * 64 + lane], lv = cur.a[(rb * 2 + 1) * 64 + lane];
      ahi[i] = v4i{static_cast<int>(hv.x), static_cast<int>(hv.y), static_cast<int>(hv.z), static_cast<int>(hv.w)};
      alo[i] = v4i{static_cast<int>(lv.x), static_cast<int>(lv.y), static_cast<int>(lv.z), static_cast<int>(lv.w)};
    }
#pragma unroll
    for (int j = 0; j < 2; j++) {
      const uint4 w = cur.b[(wn * 2 + j) * 64 + lane];
      b[j] = v4i{static_cast<int>(w.x), static_cast<int>(w.y), static_cast<int>(w.z), static_cast<int>(w.w)};
    }
    int32_t ws[2];
    float swv[2];
#pragma unroll
    for (int j = 0; j < 2; j++) {
      const int c = (wn * 2 + j) * 16 + col_in;
      ws[j] = cur.wsum[c];
      swv[j] = cur.sw[c];
    }
    float sa[RW][4];
#pragma unroll
    for (int i = 0; i < RW; i++) {
      const float4 sv = *reinterpret_cast<const float4 *>(&cur.steps[(wm * RW + i) * 16 + 4 * quad]);
      sa[i][0] = sv.x;
      sa[i][1] = sv.y;
      sa[i][2] = sv.z;
      sa[i][3] = sv.w;
    }
    const v4i zero = {0, 0, 0, 0};
#pragma unroll
    for (int i = 0; i < RW; i++)
#pragma unroll
      for (int j = 0; j < 2; j++) {
        const v4i hsum = __builtin_amdgcn_mfma_i32_16x16x64_i8(ahi[i], b[j], zero, 0, 0, 0);
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
  issue(ring0, 0);
  int g = 0;
  for (; g + 2 <= groups; g += 2) {
    step(ring0, ring1, g);
    step(ring1, ring0, g + 1);
  }
  if (g < groups) step(ring0, ring1, g);
  // The repeated copies must land before the workgroup's LDS is released.
  __builtin_amdgcn_s_waitcnt(0x0070);  // vmcnt(0) lgkmcnt(0)

  // Exception FMAs (ascending columns), then the epilogue.
#pragma unroll
  for (int i = 0; i < RW; i++) {
    const int row_base = (mb0 + wm * RW + i) * 16 + 4 * quad;
#pragma unroll
    for (int j = 0; j < 2; j++) {
      const int col = (nb0 + wn * 2 + j) * 16 + col_in;
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
  const size_t m_pad = (m + kMPad - 1) / kMPad * kMPad;
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
  // 128-column tiles where n gives at least 16 of them (fewer operand bytes
  // per output: +5 % on 1024 -> 4096), 64-column ones for narrow outputs
  // (n = 768: the wider tiles leave too few workgroups).
  const int row_tiles = static_cast<int>(m_pad / kBM);
#define FOCR_LAUNCH_I16(E, BN)                                                                                    \
  hipLaunchKernelGGL((gemm_kernel<E, BN>), dim3(static_cast<unsigned>(row_tiles * ((n + BN - 1) / BN))), dim3(BN * 4), \
                     0, ctx->stream, a_tiles, steps, exc_inputs, lin->i16_b, lin->i16_wsum, lin->i16_sw,             \
                     lin->exc_vals, static_cast<int>(lin->n_exc), static_cast<int>(m), static_cast<int>(n),          \
                     static_cast<int>(groups), static_cast<int>(row_blocks), static_cast<int>(m_pad), row_tiles,     \
                     static_cast<int>((n + BN - 1) / BN), out)
  const bool wide = n >= 2048;
  if (epilogue == FOCR_EPI_GLU) {
    if (wide) FOCR_LAUNCH_I16(FOCR_EPI_GLU, 128); else FOCR_LAUNCH_I16(FOCR_EPI_GLU, 64);
  } else if (epilogue == FOCR_EPI_ADD) {
    if (wide) FOCR_LAUNCH_I16(FOCR_EPI_ADD, 128); else FOCR_LAUNCH_I16(FOCR_EPI_ADD, 64);
  } else {
    if (wide) FOCR_LAUNCH_I16(FOCR_EPI_STORE, 128); else FOCR_LAUNCH_I16(FOCR_EPI_STORE, 64);
  }
#undef FOCR_LAUNCH_I16
  FOCR_HIP_CHECK(hipGetLastError());
  return FOCR_OK;
}

}  // namespace focr
