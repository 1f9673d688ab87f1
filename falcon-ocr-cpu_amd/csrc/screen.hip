// Exact greedy selection over the vocabulary head through an INT8 screen
// (src/head_screen.rs).
//
// The FP32 head stays authoritative. The screen (64-channel groups, RTN codes
// against absmax/127 scales) gives every vocabulary row v an approximate
// logit q_v and a bound B_v = kappa * S_v + 2^-100 with S_v = sum_g s_g n_g,
// such that |L_v - q_v| <= B_v for the FP32 logit L_v of any summation order.
// With tau = max_v (q_v - B_v), every row whose logit can reach the maximum
// has q_v + B_v >= tau; those candidates are recomputed with the reference
// dot (src/simd.rs:749-777) and the first index of the largest logit is the
// token: the full head's argmax, ties included. More than 1024 candidates, a
// non-finite or huge input, or a non-finite candidate logit is a fallback
// (the caller evaluates the full head).
//
// Two launches per call, all rows (at most 8) together:
//  1. screen_kernel: up to 768 workgroups stride over tiles of 16 vocabulary
//     rows, 16 lanes per row (lane 4g + row: 64-channel group g, 64 codes in four
//     16-byte loads, the next tile's issued before this one is scored), every
//     input scored against each row as it is loaded. The order is the reference's AVX2
//     screen_row (two 8-lane FMA chains per group, (a0 + a1) * s_g accumulated
//     lane-wise over the groups, the AVX2 horizontal sum; S by one FMA chain),
//     so q, S, the bounds and the candidate set are bit for bit the
//     reference's. Writes q + B per row and the workgroup's largest q - B.
//  2. select_kernel: one workgroup per input gathers the rows with
//     q + B >= tau, computes their FP32 logits in the reference dot order
//     and picks the largest logit with the smallest index, writing the
//     result into mapped host memory.
// HBM roofline: the screen reads vocab * (dim + 4 dim / 64) bytes once per
// call (50.3 MB for 65,536 x 768), plus 4 dim bytes per candidate.
#include <cmath>
#include <cstring>
#include <vector>

#include "focr_internal.hpp"

namespace focr {
namespace {

constexpr int kGroup = 64;
constexpr int kMaxGroups = 16;     // dim <= 1024: one lane per group, 16 lanes per row
constexpr int kLimit = 1024;       // CANDIDATE_LIMIT
constexpr int kMaxRows = 8;        // MAX_ROWS
constexpr int kRowsPerBlock = 16;  // screen rows per tile (4 waves x 4)
constexpr int kScreenBlocks = 768;  // screen workgroups (3 per compute unit at its register use)
constexpr float kEta = 7.888609e-31f;  // 2^-100

}  // namespace

struct Screen {
  size_t vocab = 0, dim = 0, groups = 0, blocks = 0, ustride = 0;
  float weight_abs_max = 0.0f, kappa = 0.0f;
  int8_t *codes = nullptr;   // [vocab][dim]
  float *scales = nullptr;   // [vocab][groups]
  // Per-call state for up to kMaxRows inputs, allocated with the screen so a
  // selection allocates nothing.
  float *upper = nullptr;      // [rows][ustride]: q + B
  float *block_max = nullptr;  // [rows][blocks]: largest q - B of each workgroup
  uint32_t *words = nullptr;   // [rows][4]: word 2 = prepare's verdict
  // [rows][2] (token, -1 = fallback; candidates) in pinned, mapped host
  // memory, written by the device through result_dev.
  int32_t *host_result = nullptr, *result_dev = nullptr;
};

namespace {

struct ScreenArgs {
  const int8_t *codes;
  const float *scales;
  const float *x;  // [rows][dim]
  const float *head;  // FP32 head [vocab][dim]
  float *upper, *block_max;
  uint32_t *words;
  int32_t *result;
  int vocab, dim, groups, rows, blocks;
  int ustride;  // row stride of upper: vocab rounded up to a multiple of 4
  float weight_abs_max, kappa;
};

// The same sum over the lanes p = lane / 4 < 8 of the screen kernel's lane
// map (lane = 4 * group + row): p ^ 4, p ^ 1, p ^ 2 are lane ^ 16, ^ 4, ^ 8.
__device__ __forceinline__ float sum8_stride4(float v) {
  v = v + __shfl_xor(v, 16, 32);
  v = v + __shfl_xor(v, 4, 32);
  v = v + __shfl_xor(v, 8, 32);
  return v;
}

__device__ __forceinline__ float sum8_lanes(float v, int p) {
  // ((v0+v4)+(v1+v5))+((v2+v6)+(v3+v7)) over lanes p = 0..7 of a row group;
  // the partner values come by exchange, and a + b = b + a exactly.
  v = v + __shfl_xor(v, 4, 8);
  v = v + __shfl_xor(v, 1, 8);
  v = v + __shfl_xor(v, 2, 8);
  return v;
}

// Dynamic LDS of screen_kernel: x [rows][groups][68] (each 64-channel group
// padded by 16 bytes, so neighbouring groups start in different banks; the
// four lanes of a group read the same address), then the per-(input of a
// pair, wave, group, row) lane values u [2][4][16][4][8] and scales
// [4][16][4] (consecutive lanes,
// consecutive words), then norms [rows][16] and the per-(row, wave) maxima
// [rows][4].
constexpr int kXPitch = kGroup + 4;
__host__ __device__ inline size_t screen_lds_bytes(int rows, int dim) {
  return sizeof(float) * (static_cast<size_t>(rows) * (dim / kGroup) * kXPitch + 2 * 4 * 4 * kMaxGroups * 8 +
                          4 * 4 * kMaxGroups + rows * kMaxGroups + rows * 4);
}

__global__ __launch_bounds__(256) void screen_kernel(ScreenArgs a) {
  extern __shared__ float lds[];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int dim = a.dim, groups = a.groups, rows = a.rows;
  const int xrow = groups * kXPitch;                    // floats per staged input row
  float *xs = lds;                                      // [rows][groups][kXPitch]
  float(*u)[4][kMaxGroups][4][8] = reinterpret_cast<float(*)[4][kMaxGroups][4][8]>(xs + rows * xrow);
  float(*sc)[kMaxGroups][4] = reinterpret_cast<float(*)[kMaxGroups][4]>(xs + rows * xrow + 2 * 4 * 4 * kMaxGroups * 8);
  float *norms = xs + rows * xrow + 2 * 4 * 4 * kMaxGroups * 8 + 4 * 4 * kMaxGroups;  // [rows][16]
  float *wmax = norms + rows * kMaxGroups;                  // [rows][4]

  // The first `rows` workgroups run prepare's input checks instead (all
  // finite; the overflow guard on the f64 L1 norm summed in ascending order)
  // and clear the later kernels' counters, while the others screen.
  if (static_cast<int>(blockIdx.x) < rows) {
    const int r = blockIdx.x;
    for (int i = tid; i < dim / 4; i += 256)
      reinterpret_cast<float4 *>(xs)[i] = reinterpret_cast<const float4 *>(a.x + static_cast<size_t>(r) * dim)[i];
    __syncthreads();
    if (tid == 0) {
      bool ok = true;
      double l1 = 0.0;
      for (int i = 0; i < dim; i += 8) {
        const float4 p0 = reinterpret_cast<const float4 *>(xs + i)[0], p1 = reinterpret_cast<const float4 *>(xs + i)[1];
        const float v8[8] = {p0.x, p0.y, p0.z, p0.w, p1.x, p1.y, p1.z, p1.w};
#pragma unroll
        for (int k = 0; k < 8; k++) {
          ok = ok && __builtin_isfinite(v8[k]);
          l1 += static_cast<double>(fabsf(v8[k]));
        }
      }
      if (ok && l1 * static_cast<double>(a.weight_abs_max) * 1.01 >= static_cast<double>(3.40282347e38f) / 2.0)
        ok = false;
      a.words[4 * r + 2] = ok ? 1u : 0u;
    }
    return;
  }
  // Screen workgroup `block` takes tiles block, block + G, ... of 16 rows (4
  // waves x 4 rows); the next tile's codes are loaded while this one is
  // scored, and the staging of x and the norms happens once.
  const int block = blockIdx.x - rows, nblocks = gridDim.x - rows;
  const int tiles = (a.vocab + kRowsPerBlock - 1) / kRowsPerBlock;
  // Lane = 4 * group + row: the four rows' lanes of a group are neighbours,
  // so their reads of the same x address share one LDS access.
  const int row_in_wave = lane & 3, g = lane >> 2;
  uint4 raw[4];
  float scale = 0.0f;
  auto load_tile = [&](int tile) {
    const int v = tile * kRowsPerBlock + wave * 4 + row_in_wave;
    if (tile < tiles && v < a.vocab && g < groups) {
      const uint4 *src = reinterpret_cast<const uint4 *>(a.codes + static_cast<size_t>(v) * dim + g * kGroup);
#pragma unroll
      for (int i = 0; i < 4; i++) raw[i] = src[i];
      scale = a.scales[static_cast<size_t>(v) * groups + g];
    } else {
#pragma unroll
      for (int i = 0; i < 4; i++) raw[i] = make_uint4(0, 0, 0, 0);
      scale = 0.0f;
    }
  };
  load_tile(block);
  for (int i = tid; i < rows * dim / 4; i += 256) {
    const int r = (4 * i) / dim, c = (4 * i) % dim;
    *reinterpret_cast<float4 *>(xs + r * xrow + (c / kGroup) * kXPitch + c % kGroup) =
        reinterpret_cast<const float4 *>(a.x)[i];
  }
  __syncthreads();
  // prepare's per-group L1 norms: exact f64 sums in ascending order, rounded up.
  // Groups past the last are zero (norm 0, scale 0, lane values 0): their
  // steps fma(0, 0, acc) leave the chains unchanged (acc is never -0), so the
  // chains below run a fixed 16 steps without branches.
  if (tid < rows * kMaxGroups) {
    const int r = tid / kMaxGroups, gg = tid % kMaxGroups;
    float n = 0.0f;
    if (gg < groups) {
      double exact = 0.0;
#pragma unroll 16
      for (int i = 0; i < kGroup; i++) exact += static_cast<double>(fabsf(xs[r * xrow + gg * kXPitch + i]));
      const float rounded = static_cast<float>(exact);
      // next_up of a finite rounded >= 0: the next bit pattern.
      n = static_cast<double>(rounded) < exact ? __uint_as_float(__float_as_uint(rounded) + 1u) : rounded;
    }
    norms[r * kMaxGroups + gg] = n;
  }
  __syncthreads();
  float wave_lower[kMaxRows];
#pragma unroll
  for (int r = 0; r < kMaxRows; r++) wave_lower[r] = -__builtin_inff();

  for (int tile = block; tile < tiles; tile += nblocks) {
    const int v = tile * kRowsPerBlock + wave * 4 + row_in_wave;
    const bool live = v < a.vocab;
    const bool active = live && g < groups;
    // This tile's codes as floats (once for every input), then the next
    // tile's loads go out.
    float cf[kGroup];
#pragma unroll
    for (int i = 0; i < kGroup; i += 4) {
      const uint32_t word = (&raw[i >> 4].x)[(i >> 2) & 3];
      cf[i] = sdwa_cvt<0>(word);
      cf[i + 1] = sdwa_cvt<1>(word);
      cf[i + 2] = sdwa_cvt<2>(word);
      cf[i + 3] = sdwa_cvt<3>(word);
    }
    sc[wave][g][row_in_wave] = scale;
    load_tile(tile + nblocks);
    // The row's 16 group scales, read once for every input (lanes g < 8 use
    // them; the write above is this wave's own and is waited for here).
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    float ss[kMaxGroups];
#pragma unroll
    for (int gg = 0; gg < kMaxGroups; gg++) ss[gg] = sc[wave][gg][row_in_wave];

    // screen_row's group step for input r into LDS slice `half`: a0 over
    // x[base + j + p], a1 over x[base + j + 8 + p], j = 0, 16, 32, 48; then
    // a0 + a1 per lane p.
    auto products = [&](int r, int half) {
      float4 *dst = reinterpret_cast<float4 *>(u[half][wave][g][row_in_wave]);
      if (!active) {
        dst[0] = dst[1] = make_float4(0.f, 0.f, 0.f, 0.f);
        return;
      }
      const float4 *xg = reinterpret_cast<const float4 *>(xs + r * xrow + g * kXPitch);
      float a0[8], a1[8];
#pragma unroll
      for (int p = 0; p < 8; p++) a0[p] = a1[p] = 0.0f;
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const float4 x0 = xg[4 * j], x1 = xg[4 * j + 1], x2 = xg[4 * j + 2], x3 = xg[4 * j + 3];
        const float xa[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
        const float xb[8] = {x2.x, x2.y, x2.z, x2.w, x3.x, x3.y, x3.z, x3.w};
#pragma unroll
        for (int p = 0; p < 8; p++) {
          a0[p] = __builtin_fmaf(xa[p], cf[16 * j + p], a0[p]);
          a1[p] = __builtin_fmaf(xb[p], cf[16 * j + 8 + p], a1[p]);
        }
      }
      dst[0] = make_float4(a0[0] + a1[0], a0[1] + a1[1], a0[2] + a1[2], a0[3] + a1[3]);
      dst[1] = make_float4(a0[4] + a1[4], a0[5] + a1[5], a0[6] + a1[6], a0[7] + a1[7]);
    };
    // Inputs go in pairs: both inputs' products, then lanes g < 8 finish
    // input r0 and lanes g >= 8 input r0 + 1 (each a 32-lane half of the
    // wave), so the exchange and its waits happen once per pair.
    for (int r0 = 0; r0 < rows; r0 += 2) {
      products(r0, 0);
      if (r0 + 1 < rows) products(r0 + 1, 1);
      // The row's 16 lanes exchange through this wave's own LDS slices.
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      const int half = g >> 3, p = g & 7;
      const int r = r0 + half;
      if (live && r < rows) {
        // Lane p accumulates row[p] = fma(a0 + a1, s_g, row[p]) over the
        // groups; S = sum fma(s_g, n_g, S) alongside.
        float uu[kMaxGroups];
#pragma unroll
        for (int gg = 0; gg < kMaxGroups; gg++) uu[gg] = u[half][wave][gg][row_in_wave][p];
        float acc = 0.0f, total = 0.0f;
#pragma unroll
        for (int gg = 0; gg < kMaxGroups; gg++) {
          acc = __builtin_fmaf(uu[gg], ss[gg], acc);
          total = __builtin_fmaf(ss[gg], norms[r * kMaxGroups + gg], total);
        }
        const float q = sum8_stride4(acc);  // within this lane's 32-lane half
        const float bound = __builtin_fmaf(a.kappa, total, kEta);
        if (p == 0) {
          a.upper[static_cast<size_t>(r) * a.ustride + v] = q + bound;
          // f32::max: a NaN operand is ignored. (Indexed by the pair's
          // uniform r0, so the array stays in registers.)
          if (half == 0)
            wave_lower[r0] = __builtin_fmaxf(wave_lower[r0], q - bound);
          else
            wave_lower[r0 + 1] = __builtin_fmaxf(wave_lower[r0 + 1], q - bound);
        }
      }
      // The next pair's products overwrite these slices only after every
      // lane has read them.
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
  }
  // The workgroup's largest q - B per input.
  for (int r = 0; r < rows; r++) {
    float m = wave_lower[r];
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) m = __builtin_fmaxf(m, __shfl_xor(m, off));
    if (lane == 0) wmax[r * 4 + wave] = m;
  }
  __syncthreads();
  if (tid < rows) {
    float m = -__builtin_inff();
    for (int w = 0; w < 4; w++) m = __builtin_fmaxf(m, wmax[tid * 4 + w]);
    a.block_max[static_cast<size_t>(tid) * a.blocks + block] = m;
  }
}

// The reference dot of x and one FP32 head row: 32 phase lanes (a0..a3 of
// eight lanes each) over the full 32-blocks, (a0 + a1) + (a2 + a3), the
// 8-wide tail, the AVX2 horizontal sum, then the unfused scalar tail.
__device__ float reference_dot(const float *x, const float *w, int len, int lane) {
  const int full = len / 32;  // at most 32 (len <= 1024)
  // Every load is issued before the FMA chain that consumes them.
  float xv[32], wv[32];
#pragma unroll
  for (int b = 0; b < 32; b++) {
    const bool in = b < full && lane < 32;
    xv[b] = in ? x[32 * b + lane] : 0.0f;
    wv[b] = in ? w[32 * b + lane] : 0.0f;
  }
  float acc = 0.0f;
#pragma unroll
  for (int b = 0; b < 32; b++)
    if (b < full) acc = __builtin_fmaf(xv[b], wv[b], acc);
  // Lane q < 8: (acc_q + acc_{q+8}) + (acc_{q+16} + acc_{q+24}).
  const float s1 = acc + __shfl_down(acc, 8, 64);
  float s = s1 + __shfl_down(s1, 16, 64);
  int i = 32 * full;
  for (; i + 8 <= len; i += 8)
    if (lane < 8) s = __builtin_fmaf(x[i + lane], w[i + lane], s);
  float total = sum8_lanes(lane < 8 ? s : 0.0f, lane & 7);
  total = __shfl(total, 0, 64);
  for (; i < len; i++) total = total + __fmul_rn(x[i], w[i]);
  return total;
}

// One workgroup per input: tau = the largest q - B (from the screen's
// workgroup maxima); the rows with q + B >= tau are gathered into an LDS list
// (one slot counter update per wave); then wave w computes the FP32 logits of
// list entries w, w + 16, ... and keeps the largest with the smallest row, and
// the workgroup combines the waves. The reference visits candidates in
// ascending order with a strict >, i.e. the first index of the maximum; more
// than kLimit candidates, a non-finite tau or a non-finite logit fall back.
__global__ __launch_bounds__(1024) void select_kernel(ScreenArgs a) {
  __shared__ float red[16];
  __shared__ uint32_t list[kLimit];
  __shared__ uint32_t count_s;
  __shared__ float best_v[16];
  __shared__ uint32_t best_i[16];
  __shared__ int bad[16];
  const int r = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  float m = -__builtin_inff();
  for (int b = tid; b < a.blocks; b += 1024) m = __builtin_fmaxf(m, a.block_max[static_cast<size_t>(r) * a.blocks + b]);
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) m = __builtin_fmaxf(m, __shfl_xor(m, off));
  if (lane == 0) red[wave] = m;
  if (tid == 0) count_s = 0;
  __syncthreads();
  float tau = -__builtin_inff();
  for (int w = 0; w < 16; w++) tau = __builtin_fmaxf(tau, red[w]);
  const bool ok = a.words[4 * r + 2] != 0 && __builtin_isfinite(tau);
  if (ok) {
    const float *upper = a.upper + static_cast<size_t>(r) * a.ustride;
    // Chunks of 64 Ki rows: every thread's 16 float4 loads go out first.
    for (int base = 0; base < a.vocab; base += 16 * 4096) {
      float4 val[16];
#pragma unroll
      for (int i = 0; i < 16; i++) {
        const int v0 = base + 4 * (1024 * i + tid);
        if (v0 + 3 < a.vocab) {
          val[i] = *reinterpret_cast<const float4 *>(upper + v0);
        } else {
          float t[4];
#pragma unroll
          for (int e = 0; e < 4; e++) t[e] = v0 + e < a.vocab ? upper[v0 + e] : -__builtin_inff();
          val[i] = make_float4(t[0], t[1], t[2], t[3]);
        }
      }
#pragma unroll
      for (int i = 0; i < 16; i++)
#pragma unroll
        for (int e = 0; e < 4; e++) {
          const int v = base + 4 * (1024 * i + tid) + e;
          const bool hit = v < a.vocab && (&val[i].x)[e] >= tau;
          const uint64_t hits = __ballot(hit);
          if (hits == 0) continue;
          const int first = __builtin_ctzll(hits);
          uint32_t slot0 = 0;
          if (lane == first) slot0 = atomicAdd(&count_s, static_cast<uint32_t>(__builtin_popcountll(hits)));
          slot0 = __shfl(slot0, first);
          if (hit) {
            const uint32_t slot =
                slot0 + static_cast<uint32_t>(__builtin_popcountll(hits & ((uint64_t(1) << lane) - 1)));
            if (slot < static_cast<uint32_t>(kLimit)) list[slot] = static_cast<uint32_t>(v);
          }
        }
    }
  }
  __syncthreads();
  const uint32_t count = count_s;
  const bool run = ok && count <= static_cast<uint32_t>(kLimit);
  float bv = -__builtin_inff();
  uint32_t bi = 0xffffffffu;
  int nonfinite = 0;
  if (run)
    for (uint32_t c = wave; c < count; c += 16) {
      const uint32_t row = list[c];
      const float l =
          reference_dot(a.x + static_cast<size_t>(r) * a.dim, a.head + static_cast<size_t>(row) * a.dim, a.dim, lane);
      if (!__builtin_isfinite(l)) nonfinite = 1;
      if (l > bv || (l == bv && row < bi)) {
        bv = l;
        bi = row;
      }
    }
  if (lane == 0) {
    best_v[wave] = bv;
    best_i[wave] = bi;
    bad[wave] = nonfinite;
  }
  __syncthreads();
  if (tid != 0) return;
  int32_t token = -1, reported = 0;
  if (ok && count > static_cast<uint32_t>(kLimit)) {
    reported = kLimit + 1;
  } else if (run && count > 0) {
    float fv = -__builtin_inff();
    uint32_t fi = 0xffffffffu;
    int anybad = 0;
    for (int w = 0; w < 16; w++) {
      anybad |= bad[w];
      if (best_v[w] > fv || (best_v[w] == fv && best_i[w] < fi)) {
        fv = best_v[w];
        fi = best_i[w];
      }
    }
    if (!anybad && fi != 0xffffffffu) {
      token = static_cast<int32_t>(fi);
      reported = static_cast<int32_t>(count);
    }
  }
  a.result[2 * r] = token;
  a.result[2 * r + 1] = reported;
}

// ScreenedHead::build's quantizer (quantize_row, src/head_screen.rs:328-366):
// returns the row's largest |w|, or a negative value if a premise fails.
float quantize_row(const float *row, size_t dim, int8_t *codes, float *scales) {
  float row_max = 0.0f;
  for (size_t g = 0; g < dim / kGroup; g++) {
    const float *values = row + g * kGroup;
    float maximum = 0.0f;
    for (int i = 0; i < kGroup; i++) {
      if (!std::isfinite(values[i])) return -1.0f;
      maximum = std::fabs(values[i]) > maximum ? std::fabs(values[i]) : maximum;
    }
    row_max = maximum > row_max ? maximum : row_max;
    float scale = 0.0f;
    if (maximum != 0.0f) {
      scale = static_cast<float>(static_cast<double>(maximum) / 127.0);
      const float tiny = 1.40129846e-45f;
      scale = scale > tiny ? scale : tiny;
    }
    scales[g] = scale;
    const double tolerance = static_cast<double>(scale) * 0.5 * (1.0 + std::ldexp(1.0, -20));
    for (int i = 0; i < kGroup; i++) {
      int8_t c = 0;
      if (scale != 0.0f) {
        double q = std::nearbyint(static_cast<double>(values[i]) / static_cast<double>(scale));
        q = q < -127.0 ? -127.0 : (q > 127.0 ? 127.0 : q);
        c = static_cast<int8_t>(q);
      }
      codes[g * kGroup + i] = c;
      const double rec = static_cast<double>(c) * static_cast<double>(scale);
      if (!(std::fabs(static_cast<double>(values[i]) - rec) <= tolerance &&
            std::fabs(static_cast<double>(values[i])) <= 127.5 * static_cast<double>(scale) * (1.0 + std::ldexp(1.0, -20))))
        return -1.0f;
    }
  }
  return row_max;
}

// kappa of a dim-wide screen (src/head_screen.rs:99-106); NaN when >= 0.53.
float screen_kappa(size_t dim) {
  const size_t groups = dim / kGroup;
  const double u = static_cast<double>(1.1920929e-7f) / 2.0;
  auto gamma = [&](size_t n) { return static_cast<double>(n) * u / (1.0 - static_cast<double>(n) * u); };
  const double k = (0.5 * (1.0 + std::ldexp(1.0, -20)) + gamma(dim) * 127.5 * (1.0 + std::ldexp(1.0, -20)) +
                    gamma(dim + groups + 8) * 127.0) *
                       (1.0 + 1e-3) +
                   2e-3;
  if (!(k < 0.53)) return NAN;
  return std::nextafter(static_cast<float>(k), INFINITY);
}

void free_screen(Screen *s) {
  void *ptrs[] = {s->codes, s->scales, s->upper, s->block_max, s->words};
  for (void *p : ptrs)
    if (p) (void)hipFree(p);
  if (s->host_result) (void)hipHostFree(s->host_result);
}

int create_screen(Ctx *ctx, const int8_t *codes, const float *scales, size_t vocab, size_t dim, float wmax,
                  float kappa, focr_screen **out) {
  FOCR_HIP_CHECK(hipSetDevice(ctx->device));
  Screen *s = new Screen();
  s->vocab = vocab;
  s->dim = dim;
  s->groups = dim / kGroup;
  const size_t tiles = (vocab + kRowsPerBlock - 1) / kRowsPerBlock;
  s->blocks = tiles < static_cast<size_t>(kScreenBlocks) ? tiles : static_cast<size_t>(kScreenBlocks);
  s->weight_abs_max = wmax;
  s->kappa = kappa;
  auto alloc = [&](void **p, size_t bytes) { return hipMalloc(p, bytes); };
  hipError_t e = hipSuccess;
  if (e == hipSuccess) e = alloc(reinterpret_cast<void **>(&s->codes), vocab * dim);
  if (e == hipSuccess) e = alloc(reinterpret_cast<void **>(&s->scales), vocab * s->groups * sizeof(float));
  s->ustride = (vocab + 3) / 4 * 4;
  if (e == hipSuccess) e = alloc(reinterpret_cast<void **>(&s->upper), kMaxRows * s->ustride * sizeof(float));
  if (e == hipSuccess) e = alloc(reinterpret_cast<void **>(&s->block_max), kMaxRows * s->blocks * sizeof(float));
  if (e == hipSuccess) e = alloc(reinterpret_cast<void **>(&s->words), kMaxRows * 4 * sizeof(uint32_t));
  if (e == hipSuccess)
    e = hipHostMalloc(reinterpret_cast<void **>(&s->host_result), kMaxRows * 2 * sizeof(int32_t),
                      hipHostMallocMapped | hipHostMallocCoherent);
  if (e == hipSuccess) e = hipHostGetDevicePointer(reinterpret_cast<void **>(&s->result_dev), s->host_result, 0);
  if (e == hipSuccess) e = hipMemcpy(s->codes, codes, vocab * dim, hipMemcpyHostToDevice);
  if (e == hipSuccess) e = hipMemcpy(s->scales, scales, vocab * s->groups * sizeof(float), hipMemcpyHostToDevice);
  if (e != hipSuccess) {
    free_screen(s);
    delete s;
    return set_error(FOCR_E_HIP, std::string("screen upload: ") + hipGetErrorString(e));
  }
  *out = reinterpret_cast<focr_screen *>(s);
  return FOCR_OK;
}

}  // namespace
}  // namespace focr

using namespace focr;

extern "C" {

int focr_screen_build(focr_ctx *handle, const float *weights, size_t vocab, size_t dim, focr_screen **out) {
  Ctx *ctx = reinterpret_cast<Ctx *>(handle);
  FOCR_REQUIRE(ctx && weights && out, FOCR_E_ARG, "focr_screen_build: null argument");
  *out = nullptr;
  FOCR_REQUIRE(vocab > 0 && dim > 0 && dim % kGroup == 0, FOCR_E_SHAPE,
               "screened head needs a nonempty head with 64-channel groups");
  FOCR_REQUIRE(vocab <= (size_t(1) << 31) - 1, FOCR_E_SHAPE, "screened head shape");
  FOCR_REQUIRE(dim <= static_cast<size_t>(kMaxGroups * kGroup), FOCR_E_UNSUPPORTED,
               "screened head: dim above 1024 is not supported by this backend");
  const float kappa = screen_kappa(dim);
  FOCR_REQUIRE(std::isfinite(kappa), FOCR_E_VALUE, "screened head bound is unexpectedly loose");
  const size_t groups = dim / kGroup;
  std::vector<int8_t> codes(vocab * dim);
  std::vector<float> scales(vocab * groups);
  float wmax = 0.0f;
  for (size_t r = 0; r < vocab; r++) {
    const float m = quantize_row(weights + r * dim, dim, codes.data() + r * dim, scales.data() + r * groups);
    FOCR_REQUIRE(m >= 0.0f, FOCR_E_VALUE, "screened head weights must be finite and meet the quantization premise");
    wmax = m > wmax ? m : wmax;
  }
  FOCR_REQUIRE(std::isfinite(wmax), FOCR_E_VALUE, "screened head weights must be finite");
  return create_screen(ctx, codes.data(), scales.data(), vocab, dim, wmax, kappa, out);
}

int focr_screen_upload(focr_ctx *handle, const int8_t *codes, const float *scales, size_t vocab, size_t dim,
                       float weight_abs_max, float kappa, focr_screen **out) {
  Ctx *ctx = reinterpret_cast<Ctx *>(handle);
  FOCR_REQUIRE(ctx && codes && scales && out, FOCR_E_ARG, "focr_screen_upload: null argument");
  *out = nullptr;
  FOCR_REQUIRE(vocab > 0 && dim > 0 && dim % kGroup == 0 && vocab <= (size_t(1) << 31) - 1, FOCR_E_SHAPE,
               "mapped screen shape");
  FOCR_REQUIRE(dim <= static_cast<size_t>(kMaxGroups * kGroup), FOCR_E_UNSUPPORTED,
               "screened head: dim above 1024 is not supported by this backend");
  FOCR_REQUIRE(std::isfinite(weight_abs_max) && std::isfinite(kappa) && kappa > 0.0f && kappa < 0.53f, FOCR_E_VALUE,
               "mapped screen constants");
  return create_screen(ctx, codes, scales, vocab, dim, weight_abs_max, kappa, out);
}

int focr_screen_free(focr_screen *handle) {
  Screen *s = reinterpret_cast<Screen *>(handle);
  if (!s) return FOCR_OK;
  free_screen(s);
  delete s;
  return FOCR_OK;
}

int focr_screen_constants(const focr_screen *handle, float *weight_abs_max, float *kappa) {
  const Screen *s = reinterpret_cast<const Screen *>(handle);
  FOCR_REQUIRE(s, FOCR_E_ARG, "focr_screen_constants: null screen");
  if (weight_abs_max) *weight_abs_max = s->weight_abs_max;
  if (kappa) *kappa = s->kappa;
  return FOCR_OK;
}

int focr_screen_select(focr_ctx *handle, const focr_screen *sh, const focr_linear *head_handle, const float *x,
                       size_t rows, int32_t *tokens, uint32_t *candidates) {
  Ctx *ctx = reinterpret_cast<Ctx *>(handle);
  const Screen *s = reinterpret_cast<const Screen *>(sh);
  const Linear *head = reinterpret_cast<const Linear *>(head_handle);
  FOCR_REQUIRE(ctx && s && head && x && tokens && candidates, FOCR_E_ARG, "focr_screen_select: null argument");
  FOCR_REQUIRE(rows >= 1 && rows <= static_cast<size_t>(kMaxRows), FOCR_E_SHAPE, "screened head: 1 to 8 input rows");
  FOCR_REQUIRE(head->bits == 32 && head->n == s->vocab && head->k == s->dim && head->n_exc == 0, FOCR_E_SHAPE,
               "screened head FP32 shape");
  FOCR_HIP_CHECK(hipSetDevice(ctx->device));
  ScreenArgs a;
  a.codes = s->codes;
  a.scales = s->scales;
  a.x = x;
  a.head = static_cast<const float *>(head->codes);
  a.upper = s->upper;
  a.block_max = s->block_max;
  a.words = s->words;
  a.result = s->result_dev;
  a.vocab = static_cast<int>(s->vocab);
  a.dim = static_cast<int>(s->dim);
  a.groups = static_cast<int>(s->groups);
  a.rows = static_cast<int>(rows);
  a.blocks = static_cast<int>(s->blocks);
  a.ustride = static_cast<int>(s->ustride);
  a.weight_abs_max = s->weight_abs_max;
  a.kappa = s->kappa;
  hipLaunchKernelGGL(screen_kernel, dim3(a.blocks + a.rows), dim3(256), screen_lds_bytes(a.rows, a.dim), ctx->stream,
                     a);
  hipLaunchKernelGGL(select_kernel, dim3(a.rows), dim3(1024), 0, ctx->stream, a);
  FOCR_HIP_CHECK(hipGetLastError());
  // select_kernel wrote the results straight into the mapped host buffer.
  FOCR_HIP_CHECK(hipStreamSynchronize(ctx->stream));
  const volatile int32_t *result = s->host_result;
  for (size_t r = 0; r < rows; r++) {
    tokens[r] = result[2 * r];
    candidates[r] = static_cast<uint32_t>(result[2 * r + 1]);
  }
  return FOCR_OK;
}

}  // extern "C"
