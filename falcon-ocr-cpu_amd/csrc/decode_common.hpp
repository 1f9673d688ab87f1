// Pieces shared by the decode attention kernels (compact cache and sealed
// split records): lane reductions, the online-softmax state merge and the
// kernel that combines the split-K partial states of every (row, head).
#pragma once

#include "focr_internal.hpp"

namespace focr {
namespace decode {

constexpr int kWaves = 4;  // waves per workgroup

template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}

// Sum over the 16 lanes of a DPP row; every lane of the row gets the same
// value (each step adds a value and its mirror image, so partners agree).
__device__ __forceinline__ float row_sum16(float v) {
  v = v + dpp<0xB1>(v);   // quad_perm [1,0,3,2]
  v = v + dpp<0x4E>(v);   // quad_perm [2,3,0,1]
  v = v + dpp<0x141>(v);  // row_half_mirror
  return v + dpp<0x140>(v);  // row_mirror
}

__device__ __forceinline__ float xor_lane(float x, int mask) {
  const int lane = threadIdx.x & 63;
  return __int_as_float(__builtin_amdgcn_ds_bpermute((lane ^ mask) << 2, __float_as_int(x)));
}

// rms_norm_row (width 64, no weight, eps f32::EPSILON) then the pairwise
// RoPE rotation for the head whose element `lane` is x (split_norm_rope and
// fused_row, src/model/rope.rs:60-72, src/model/fused.rs:107-120): the
// 64-wide pairwise sum of squares is two 32-leaves folded 16-8-4-2-1 (xor
// butterflies) then leaf0 + leaf1; scale = 1 / sqrt(sum / 64 + eps) with IEEE
// division and square root; separate roundings, no contraction. Returns the
// rotated element.
__device__ __forceinline__ float norm_rope(float x, float2 factor, int lane) {
  float part = x * x;
#pragma unroll
  for (int w = 16; w >= 1; w /= 2) part = part + xor_lane(part, w);
  const float leaf0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(part), 0));
  const float leaf1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(part), 32));
  const float sum = leaf0 + leaf1;
  const float scale = __fdiv_rn(1.0f, __builtin_sqrtf(__fdiv_rn(sum, 64.0f) + 1.1920929e-7f));
  const float y = x * scale;
  const float partner = xor_lane(y, 1);
  const bool even = (lane & 1) == 0;
  const float a = even ? y : partner, b = even ? partner : y;
  return even ? a * factor.x - b * factor.y : a * factor.y + b * factor.x;
}

__device__ __forceinline__ float4 ld4(const float *p) { return *reinterpret_cast<const float4 *>(p); }

// Merge two online-softmax states (max m, denominator d, output o); both
// partners compute the same bits (products identical, sums commutative).
__device__ __forceinline__ void merge(float &m, float &d, float4 &o, float m2, float d2, float4 o2) {
  const float mn = m > m2 ? m : m2;
  if (mn == -__builtin_inff()) return;  // both empty
  const float f1 = m == -__builtin_inff() ? 0.0f : expf_acc(m - mn);
  const float f2 = m2 == -__builtin_inff() ? 0.0f : expf_acc(m2 - mn);
  d = d * f1 + d2 * f2;
  o = make_float4(o.x * f1 + o2.x * f2, o.y * f1 + o2.y * f2, o.z * f1 + o2.z * f2, o.w * f1 + o2.w * f2);
  m = mn;
}

struct CombineArgs {
  const float *part_o, *part_md, *sinks;
  float *out;
  int n_heads, chunks;
};

constexpr int kMaxChunks = 1024;

// Sum over a wave in a fixed order (every lane gets the same value).
__device__ __forceinline__ float wave_sum(float v) {
  v = row_sum16(v);
  v = v + xor_lane(v, 16);
  return v + xor_lane(v, 32);
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int mask = 1; mask < 64; mask *= 2) {
    const float o = xor_lane(v, mask);
    v = o > v ? o : v;
  }
  return v;
}

// One workgroup per (row, head). Thread t takes chunks t, t + 256, ... for
// the maximum and the weights exp(m_c - M); then lane = dim and wave w sums
// the outputs of chunks w, w + 4, ... in ascending order; the partial sums
// are added in a fixed order. The (max, den) pairs are read once, and each
// wave's first 16 output loads are issued with them, before the maximum is
// known, so the reads overlap instead of following one another. Final step
// as online.rs head (lines 144-149): lse = max + ln(den),
// out = (o / den) * 1/(1 + exp(sink - lse)).
// The work of one (row, head): a workgroup of 256 threads, `sh` its LDS.
struct CombineShared {
  float f[kMaxChunks];
  float red[kWaves], o[kWaves][64];
};
__device__ __forceinline__ void combine_row(const CombineArgs &a, int rh, CombineShared &sh) {
  constexpr int kPer = kMaxChunks / 256;  // (max, den) pairs per thread
  constexpr int kPre = 16;                // outputs per wave loaded up front
  float *s_f = sh.f;
  float *s_red = sh.red;
  float (*s_o)[64] = sh.o;
  const int h = rh % a.n_heads;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const float2 *md = reinterpret_cast<const float2 *>(a.part_md) + static_cast<size_t>(rh) * a.chunks;
  const float *po = a.part_o + static_cast<size_t>(rh) * a.chunks * 64;
  const float ninf = -__builtin_inff();
  float2 mdv[kPer];
#pragma unroll
  for (int i = 0; i < kPer; i++) {
    const int c = tid + 256 * i;
    mdv[i] = c < a.chunks ? md[c] : make_float2(ninf, 0.0f);
  }
  float ov[kPre];
#pragma unroll
  for (int i = 0; i < kPre; i++) {
    const int c = wave + 4 * i;
    ov[i] = c < a.chunks ? po[static_cast<size_t>(c) * 64 + lane] : 0.0f;
  }
  float mx = ninf;
#pragma unroll
  for (int i = 0; i < kPer; i++) mx = mdv[i].x > mx ? mdv[i].x : mx;
  mx = wave_max(mx);
  if (lane == 0) s_red[wave] = mx;
  __syncthreads();
  float big = s_red[0];
#pragma unroll
  for (int w = 1; w < kWaves; w++) big = s_red[w] > big ? s_red[w] : big;
  __syncthreads();
  float den = 0.0f;
#pragma unroll
  for (int i = 0; i < kPer; i++) {
    const int c = tid + 256 * i;
    if (c < a.chunks) {
      const float mc = mdv[i].x;
      const float f = mc == ninf || big == ninf ? 0.0f : expf_acc(mc - big);
      s_f[c] = f;
      den = den + mdv[i].y * f;
    }
  }
  den = wave_sum(den);
  if (lane == 0) s_red[wave] = den;
  __syncthreads();
  float o = 0.0f;
  int c = wave;
#pragma unroll
  for (int i = 0; i < kPre; i++, c += 4)
    if (c < a.chunks) o = fmaf_(ov[i], s_f[c], o);
  // The rest, sixteen loads in flight before their products are added (in
  // chunk order).
  for (; c + 60 < a.chunks; c += 64) {
    float v[16];
#pragma unroll
    for (int i = 0; i < 16; i++) v[i] = po[static_cast<size_t>(c + 4 * i) * 64 + lane];
#pragma unroll
    for (int i = 0; i < 16; i++) o = fmaf_(v[i], s_f[c + 4 * i], o);
  }
  for (; c < a.chunks; c += 4) o = fmaf_(po[static_cast<size_t>(c) * 64 + lane], s_f[c], o);
  s_o[wave][lane] = o;
  __syncthreads();
  if (wave == 0) {
    const float d = (s_red[0] + s_red[1]) + (s_red[2] + s_red[3]);
    const float total = (s_o[0][lane] + s_o[1][lane]) + (s_o[2][lane] + s_o[3][lane]);
    const float lse = big + logf_acc(d);
    const float sink_scale = __fdiv_rn(1.0f, 1.0f + expf_acc(a.sinks[h] - lse));
    a.out[static_cast<size_t>(rh) * 64 + lane] = __fdiv_rn(total, d) * sink_scale;
  }
  __syncthreads();  // the LDS may be reused for the next (row, head)
}

static __global__ __launch_bounds__(256) void decode_combine_kernel(CombineArgs a) {
  __shared__ CombineShared sh;
  combine_row(a, blockIdx.x, sh);
}

}  // namespace decode
}  // namespace focr
