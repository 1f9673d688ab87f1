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
//  1. screen_kernel: one workgroup per 64 vocabulary rows, lane l row 64 b + l.
//     The reference's AVX2 screen_row keeps eight phase lanes p per row: two
//     FMA chains per group (a0 over x[64 g + j + p], a1 over x[64 g + j + 8 + p],
//     j = 0, 16, 32, 48), (a0 + a1) * s_g accumulated per phase over the
//     groups, then the AVX2 horizontal sum; S by one FMA chain. Here wave w
//     runs the phases p = 2w and 2w + 1 of all 64 rows, so the x values a wave
//     needs at any step are the same for every lane: the inputs are staged in
//     LDS in the order a wave reads them, and each step's 16 values are four
//     LDS broadcast reads. The codes are stored at upload in the order one
//     wave consumes them (16 bytes per row, group and wave: one coalesced 1 KB
//     load), group-major. The four waves' phase sums meet in LDS for the
//     horizontal sum, so q, S, the bounds and the candidate set are bit for
//     bit the reference's. Writes q + B per row and the block's largest q - B
//     and q + B.
//  2. select_kernel: one workgroup per input takes tau from the blocks'
//     maxima, tests only the rows of blocks whose largest q + B reaches tau,
//     computes the candidates' FP32 logits in the reference dot order and
//     picks the largest logit with the smallest index, writing the result
//     into mapped host memory.
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
constexpr int kBlockRows = 64;     // vocabulary rows per screen workgroup (one per lane)
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
  float *block_max = nullptr;    // [rows][blocks]: largest q - B of each 64-row block
  float *block_upper = nullptr;  // [rows][blocks]: largest q + B of each 64-row block
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
  float *upper, *block_max, *block_upper;
  uint32_t *words;
  int32_t *result;
  int vocab, dim, groups, rows, blocks;
  int ustride;  // row stride of upper: vocab rounded up to a multiple of 4
  float weight_abs_max, kappa;
};

// Device layout of the screen (written at upload, rows padded to a multiple
// of 64 with zero codes and scales), group-major so that the loads every
// workgroup issues together cover one contiguous span:
//  codes  [group][block][wave][lane][16]: wave w's bytes of row 64 block +
//         lane and group g are, for j = 0, 16, 32, 48, the codes j + 2w,
//         j + 2w + 1 (chain a0 of phases 2w, 2w + 1) and j + 8 + 2w, j + 9 + 2w
//         (chain a1);
//  scales [group][block][lane].
__host__ __device__ inline size_t screen_code_offset(size_t blocks, size_t block, size_t g, int wave, int lane) {
  return (((g * blocks + block) * 4 + static_cast<size_t>(wave)) * kBlockRows + static_cast<size_t>(lane)) * 16;
}

// Staged input blocks: input r, group g at xp[(r * groups + g) * kXBlock],
// 4 padding floats after each so that lanes reading different blocks at the
// same offset use distinct LDS banks.
constexpr int kXBlock = kGroup + 4;
union ScreenLds {
  float x[kMaxGroups * kGroup];  // prepare workgroups: the staged input row
  struct {
    // The inputs in the order a wave reads them, within a block [wave][16]
    // with element 4 j + c = x[64 g + 16 j + 2 wave + (0, 1, 8, 9)[c]] (four
    // 16-byte reads per step, the same address in every lane: an LDS
    // broadcast), and prepare's norms [input][group].
    float xp[kMaxRows * kMaxGroups * kXBlock];
    float norms[kMaxRows * kMaxGroups];
  } in;
  float part[kMaxRows][8][kBlockRows];  // per input, phase, row: the phase sums
};

// ROWS inputs (1..8).
template <int ROWS>
__global__ __launch_bounds__(256) void screen_kernel(ScreenArgs a) {
  __shared__ ScreenLds lds;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int dim = a.dim, groups = a.groups;
  // The first ROWS workgroups run prepare's input checks instead (all
  // finite; the overflow guard on the f64 L1 norm summed in ascending order)
  // while the others screen.
  if (static_cast<int>(blockIdx.x) < ROWS) {
    const int r = blockIdx.x;
    float *xs = lds.x;
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
  const int block = blockIdx.x - ROWS;
  const int v = block * kBlockRows + lane;
  // The inputs for the staging, then the codes and scales of the lane's row
  // for kWindow groups (group g + kWindow's loads go out when group g is
  // converted). Thread t stages inputs' elements 4t .. 4t + 3 (dim <= 1024).
  const int k4 = 4 * tid;
  float4 xin[ROWS];
#pragma unroll
  for (int r = 0; r < ROWS; r++)
    xin[r] = k4 < dim ? *reinterpret_cast<const float4 *>(a.x + static_cast<size_t>(r) * dim + k4)
                      : make_float4(0.f, 0.f, 0.f, 0.f);
  constexpr int kWindow = 8;
  const uint4 *csrc = reinterpret_cast<const uint4 *>(a.codes + screen_code_offset(a.blocks, block, 0, wave, lane));
  const float *ssrc = a.scales + static_cast<size_t>(block) * kBlockRows + lane;
  const size_t cstride = static_cast<size_t>(a.blocks) * 4 * kBlockRows, sstride = static_cast<size_t>(a.blocks) * kBlockRows;
  uint4 raw[kWindow];
  float sg[kWindow];
#pragma unroll
  for (int u = 0; u < kWindow; u++) {
    raw[u] = u < groups ? csrc[u * cstride] : make_uint4(0, 0, 0, 0);
    sg[u] = u < groups ? ssrc[u * sstride] : 0.0f;
  }
  // Stage: elements m0 .. m0 + 3 of a 16-block (m0 = 0, 4, 8, 12) go to
  // waves w0, w0 + 1 (w0 = 0 or 2), slots c0, c0 + 1 (c0 = 0 or 2).
  if (k4 < dim) {
    const int g = k4 / kGroup, j = (k4 % kGroup) / 16, m0 = k4 % 16;
    const int w0 = (m0 & 4) >> 1, c0 = (m0 >> 3) << 1;
#pragma unroll
    for (int r = 0; r < ROWS; r++) {
      float *dst = lds.in.xp + (r * groups + g) * kXBlock + w0 * 16 + 4 * j + c0;
      *reinterpret_cast<float2 *>(dst) = make_float2(xin[r].x, xin[r].y);
      *reinterpret_cast<float2 *>(dst + 16) = make_float2(xin[r].z, xin[r].w);
    }
  }
  // Plain barriers: LDS writes complete (lgkmcnt(0)); the code loads stay in
  // flight.
  auto lds_barrier = []() __attribute__((always_inline)) {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xc07f);
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
  };
  lds_barrier();
  // prepare's per-group L1 norms (exact f64 sums in ascending order, rounded
  // up): thread 16 r + g, from the staged block. x[64 g + 16 j + m] sits in
  // the wave (m & 7) / 2 slice at 4 j + (m & 1) + 2 (m >> 3).
  if (tid < ROWS * kMaxGroups) {
    const int r = tid / kMaxGroups, g = tid % kMaxGroups;
    float n = 0.0f;
    if (g < groups) {
      const float *blk = lds.in.xp + (r * groups + g) * kXBlock;
      double exact = 0.0;
#pragma unroll
      for (int j = 0; j < 4; j++) {
        float4 q[4];
#pragma unroll
        for (int w = 0; w < 4; w++) q[w] = *reinterpret_cast<const float4 *>(blk + 16 * w + 4 * j);
#pragma unroll
        for (int w = 0; w < 4; w++) {  // m = 2w, 2w + 1
          exact += static_cast<double>(fabsf(q[w].x));
          exact += static_cast<double>(fabsf(q[w].y));
        }
#pragma unroll
        for (int w = 0; w < 4; w++) {  // m = 8 + 2w, 9 + 2w
          exact += static_cast<double>(fabsf(q[w].z));
          exact += static_cast<double>(fabsf(q[w].w));
        }
      }
      const float rounded = static_cast<float>(exact);
      // next_up of a finite rounded >= 0: the next bit pattern.
      n = static_cast<double>(rounded) < exact ? __uint_as_float(__float_as_uint(rounded) + 1u) : rounded;
    }
    lds.in.norms[tid] = n;
  }
  lds_barrier();

  // Phase sums row[p] of p = 2 wave + e for every input, and S.
  float acc[ROWS][2], total[ROWS];
#pragma unroll
  for (int r = 0; r < ROWS; r++) acc[r][0] = acc[r][1] = total[r] = 0.0f;
  for (int g0 = 0; g0 < groups; g0 += kWindow) {
#pragma unroll
    for (int u = 0; u < kWindow; u++) {
      const int g = g0 + u;
      if (g >= groups) break;
      float cf[16];
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const uint32_t word = (&raw[u].x)[i];
        cf[4 * i] = sdwa_cvt<0>(word);
        cf[4 * i + 1] = sdwa_cvt<1>(word);
        cf[4 * i + 2] = sdwa_cvt<2>(word);
        cf[4 * i + 3] = sdwa_cvt<3>(word);
      }
      const float s = sg[u];
      if (g + kWindow < groups) {
        raw[u] = csrc[(g + kWindow) * cstride];
        sg[u] = ssrc[(g + kWindow) * sstride];
      }
#pragma unroll
      for (int r = 0; r < ROWS; r++) {
        const float4 *xq = reinterpret_cast<const float4 *>(lds.in.xp + (r * groups + g) * kXBlock + wave * 16);
        const float n = lds.in.norms[r * kMaxGroups + g];
        float a00 = 0.0f, a01 = 0.0f, a10 = 0.0f, a11 = 0.0f;
#pragma unroll
        for (int j = 0; j < 4; j++) {
          const float4 xv = xq[j];
          a00 = __builtin_fmaf(xv.x, cf[4 * j], a00);
          a01 = __builtin_fmaf(xv.y, cf[4 * j + 1], a01);
          a10 = __builtin_fmaf(xv.z, cf[4 * j + 2], a10);
          a11 = __builtin_fmaf(xv.w, cf[4 * j + 3], a11);
        }
        acc[r][0] = __builtin_fmaf(a00 + a10, s, acc[r][0]);
        acc[r][1] = __builtin_fmaf(a01 + a11, s, acc[r][1]);
        total[r] = __builtin_fmaf(s, n, total[r]);
      }
    }
  }
  __syncthreads();  // every wave is done with xp before part overwrites it
  // The horizontal sum ((v0 + v4) + (v1 + v5)) + ((v2 + v6) + (v3 + v7)) of
  // each input's eight phases; wave w finishes the inputs r = w, w + 4.
#pragma unroll
  for (int r = 0; r < ROWS; r++) {
    lds.part[r][2 * wave][lane] = acc[r][0];
    lds.part[r][2 * wave + 1][lane] = acc[r][1];
  }
  __syncthreads();
#pragma unroll
  for (int r = 0; r < ROWS; r++) {
    if ((r & 3) != wave) continue;
    float p8[8];
#pragma unroll
    for (int p = 0; p < 8; p++) p8[p] = lds.part[r][p][lane];
    const float q = ((p8[0] + p8[4]) + (p8[1] + p8[5])) + ((p8[2] + p8[6]) + (p8[3] + p8[7]));
    const float bound = __builtin_fmaf(a.kappa, total[r], kEta);
    // f32::max: a NaN operand is ignored. The block's largest q + B lets
    // the selection skip blocks that hold no candidate.
    float lower = -__builtin_inff(), high = -__builtin_inff();
    if (v < a.vocab) {
      const float hi = q + bound;
      a.upper[static_cast<size_t>(r) * a.ustride + v] = hi;
      lower = __builtin_fmaxf(lower, q - bound);
      high = __builtin_fmaxf(high, hi);
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
      lower = __builtin_fmaxf(lower, __shfl_xor(lower, off));
      high = __builtin_fmaxf(high, __shfl_xor(high, off));
    }
    if (lane == 0) {
      a.block_max[static_cast<size_t>(r) * a.blocks + block] = lower;
      a.block_upper[static_cast<size_t>(r) * a.blocks + block] = high;
    }
  }
}

// The same sum over eight lanes p of a row group as the reference's AVX2
// horizontal sum: ((v0+v4)+(v1+v5))+((v2+v6)+(v3+v7)), partner values by
// exchange (a + b = b + a exactly).
__device__ __forceinline__ float sum8_lanes(float v, int p) {
  v = v + __shfl_xor(v, 4, 8);
  v = v + __shfl_xor(v, 1, 8);
  v = v + __shfl_xor(v, 2, 8);
  return v;
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

// One workgroup per input: tau = the largest q - B (from the blocks'
// maxima); the 64-row blocks whose largest q + B reaches tau are listed, and
// only their rows are tested: the rows with q + B >= tau go into an LDS list
// (one slot counter update per wave). Then wave w computes the FP32 logits of
// list entries w, w + 16, ... and keeps the largest with the smallest row, and
// the workgroup combines the waves. The reference visits candidates in
// ascending order with a strict >, i.e. the first index of the maximum; more
// than kLimit candidates, a non-finite tau or a non-finite logit fall back.
__global__ __launch_bounds__(1024) void select_kernel(ScreenArgs a) {
  __shared__ float red[16];
  __shared__ uint32_t list[kLimit];
  __shared__ uint32_t hot[kLimit];
  __shared__ uint32_t count_s, hot_s;
  __shared__ float best_v[16];
  __shared__ uint32_t best_i[16];
  __shared__ int bad[16];
  const int r = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const float *bmax = a.block_max + static_cast<size_t>(r) * a.blocks;
  const float *bup = a.block_upper + static_cast<size_t>(r) * a.blocks;
  // Both block arrays' first 1024 entries are loaded together.
  const float up0 = tid < a.blocks ? bup[tid] : -__builtin_inff();
  float m = tid < a.blocks ? bmax[tid] : -__builtin_inff();
  for (int b = tid + 1024; b < a.blocks; b += 1024) m = __builtin_fmaxf(m, bmax[b]);
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) m = __builtin_fmaxf(m, __shfl_xor(m, off));
  if (lane == 0) red[wave] = m;
  if (tid == 0) count_s = hot_s = 0;
  __syncthreads();
  float tau = -__builtin_inff();
  for (int w = 0; w < 16; w++) tau = __builtin_fmaxf(tau, red[w]);
  const bool ok = a.words[4 * r + 2] != 0 && __builtin_isfinite(tau);
  // Append the lanes' hits to an LDS list: one counter update per wave.
  auto append = [&](bool hit, uint32_t value, uint32_t *dst, uint32_t *counter) {
    const uint64_t hits = __ballot(hit);
    if (hits == 0) return;
    const int first = __builtin_ctzll(hits);
    uint32_t slot0 = 0;
    if (lane == first) slot0 = atomicAdd(counter, static_cast<uint32_t>(__builtin_popcountll(hits)));
    slot0 = __shfl(slot0, first);
    if (hit) {
      const uint32_t slot = slot0 + static_cast<uint32_t>(__builtin_popcountll(hits & ((uint64_t(1) << lane) - 1)));
      if (slot < static_cast<uint32_t>(kLimit)) dst[slot] = value;
    }
  };
  if (ok) {
    // Every block that holds a candidate has its largest q + B >= tau, so
    // more than kLimit such blocks means more than kLimit candidates.
    append(tid < a.blocks && up0 >= tau, static_cast<uint32_t>(tid), hot, &hot_s);
    for (int b = tid + 1024; b - tid < a.blocks; b += 1024) append(b < a.blocks && bup[b] >= tau, b, hot, &hot_s);
  }
  __syncthreads();
  const uint32_t n_hot = hot_s;
  if (ok && n_hot <= static_cast<uint32_t>(kLimit)) {
    const float *upper = a.upper + static_cast<size_t>(r) * a.ustride;
    for (uint32_t i = wave; i < n_hot; i += 16) {
      const int v = static_cast<int>(hot[i]) * kBlockRows + lane;
      append(v < a.vocab && upper[v] >= tau, static_cast<uint32_t>(v), list, &count_s);
    }
  }
  __syncthreads();
  const uint32_t count = n_hot > static_cast<uint32_t>(kLimit) ? static_cast<uint32_t>(kLimit) + 1 : count_s;
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
  void *ptrs[] = {s->codes, s->scales, s->upper, s->block_max, s->block_upper, s->words};
  for (void *p : ptrs)
    if (p) (void)hipFree(p);
  if (s->host_result) (void)hipHostFree(s->host_result);
}

int create_screen(Ctx *ctx, const int8_t *codes, const float *scales, size_t vocab, size_t dim, float wmax,
                  float kappa, focr_screen **out) {
  FOCR_HIP_CHECK(hipSetDevice(ctx->device));
  const size_t groups = dim / kGroup;
  const size_t blocks = (vocab + kBlockRows - 1) / kBlockRows;
  // The device layout (screen_code_offset): each wave's 16 code bytes of a
  // row and group in the order its two phases consume them.
  std::vector<int8_t> dev_codes(blocks * kBlockRows * dim, 0);
  std::vector<float> dev_scales(blocks * groups * kBlockRows, 0.0f);
  for (size_t v = 0; v < vocab; v++) {
    const size_t b = v / kBlockRows;
    const int l = static_cast<int>(v % kBlockRows);
    for (size_t g = 0; g < groups; g++) {
      dev_scales[(g * blocks + b) * kBlockRows + static_cast<size_t>(l)] = scales[v * groups + g];
      const int8_t *src = codes + v * dim + g * kGroup;
      for (int w = 0; w < 4; w++) {
        int8_t *dst = dev_codes.data() + screen_code_offset(blocks, b, g, w, l);
        for (int j = 0; j < 4; j++) {
          dst[4 * j] = src[16 * j + 2 * w];
          dst[4 * j + 1] = src[16 * j + 2 * w + 1];
          dst[4 * j + 2] = src[16 * j + 8 + 2 * w];
          dst[4 * j + 3] = src[16 * j + 9 + 2 * w];
        }
      }
    }
  }
  Screen *s = new Screen();
  s->vocab = vocab;
  s->dim = dim;
  s->groups = groups;
  s->blocks = blocks;
  s->weight_abs_max = wmax;
  s->kappa = kappa;
  auto alloc = [&](void **p, size_t bytes) { return hipMalloc(p, bytes); };
  hipError_t e = hipSuccess;
  if (e == hipSuccess) e = alloc(reinterpret_cast<void **>(&s->codes), dev_codes.size());
  if (e == hipSuccess) e = alloc(reinterpret_cast<void **>(&s->scales), dev_scales.size() * sizeof(float));
  s->ustride = (vocab + 3) / 4 * 4;
  if (e == hipSuccess) e = alloc(reinterpret_cast<void **>(&s->upper), kMaxRows * s->ustride * sizeof(float));
  if (e == hipSuccess) e = alloc(reinterpret_cast<void **>(&s->block_max), kMaxRows * s->blocks * sizeof(float));
  if (e == hipSuccess) e = alloc(reinterpret_cast<void **>(&s->block_upper), kMaxRows * s->blocks * sizeof(float));
  if (e == hipSuccess) e = alloc(reinterpret_cast<void **>(&s->words), kMaxRows * 4 * sizeof(uint32_t));
  if (e == hipSuccess)
    e = hipHostMalloc(reinterpret_cast<void **>(&s->host_result), kMaxRows * 2 * sizeof(int32_t),
                      hipHostMallocMapped | hipHostMallocCoherent);
  if (e == hipSuccess) e = hipHostGetDevicePointer(reinterpret_cast<void **>(&s->result_dev), s->host_result, 0);
  if (e == hipSuccess) e = hipMemcpy(s->codes, dev_codes.data(), dev_codes.size(), hipMemcpyHostToDevice);
  if (e == hipSuccess)
    e = hipMemcpy(s->scales, dev_scales.data(), dev_scales.size() * sizeof(float), hipMemcpyHostToDevice);
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

int focr_screen_bounds(const focr_screen *handle, size_t rows, float *upper_host) {
  const Screen *s = reinterpret_cast<const Screen *>(handle);
  FOCR_REQUIRE(s && upper_host, FOCR_E_ARG, "focr_screen_bounds: null argument");
  FOCR_REQUIRE(rows >= 1 && rows <= static_cast<size_t>(kMaxRows), FOCR_E_SHAPE, "screened head: 1 to 8 input rows");
  for (size_t r = 0; r < rows; r++)
    FOCR_HIP_CHECK(hipMemcpy(upper_host + r * s->vocab, s->upper + r * s->ustride, s->vocab * sizeof(float),
                             hipMemcpyDeviceToHost));
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
  a.block_upper = s->block_upper;
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
  const dim3 grid(static_cast<unsigned>(a.blocks + a.rows));
  switch (rows) {
    case 1: hipLaunchKernelGGL(screen_kernel<1>, grid, dim3(256), 0, ctx->stream, a); break;
    case 2: hipLaunchKernelGGL(screen_kernel<2>, grid, dim3(256), 0, ctx->stream, a); break;
    case 3: hipLaunchKernelGGL(screen_kernel<3>, grid, dim3(256), 0, ctx->stream, a); break;
    case 4: hipLaunchKernelGGL(screen_kernel<4>, grid, dim3(256), 0, ctx->stream, a); break;
    case 5: hipLaunchKernelGGL(screen_kernel<5>, grid, dim3(256), 0, ctx->stream, a); break;
    case 6: hipLaunchKernelGGL(screen_kernel<6>, grid, dim3(256), 0, ctx->stream, a); break;
    case 7: hipLaunchKernelGGL(screen_kernel<7>, grid, dim3(256), 0, ctx->stream, a); break;
    default: hipLaunchKernelGGL(screen_kernel<8>, grid, dim3(256), 0, ctx->stream, a); break;
  }
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
