// rms_scale (src/kernels/mod.rs:531-553) for widths known at compile time:
// 1 / sqrt(sum_squares_pairwise(x) / width + eps), IEEE division and sqrt.
//
// sum_squares_pairwise splits a segment of len > 32 values at
// (len / 2).next_multiple_of(32) and adds left + right; a segment of at most
// 32 values squares them into 32 zero-padded slots and folds
// partial[i] += partial[i + w] for w = 16, 8, 4, 2, 1. Every split point is a
// multiple of 32 from a segment start that is itself one, so the leaves are
// the consecutive 32-chunks of the row (the last one possibly shorter); only
// the order in which leaves are added depends on the width. PairTree<LEN>
// unrolls that order at compile time, so a wave computes the leaves in
// parallel (lane i: leaves i, i + 64, ...) and adds them in the reference's
// order in straight-line code.
#pragma once

#include "focr_internal.hpp"

namespace focr {

template <int LEN, bool LEAF = (LEN <= 32)>
struct PairTree;

template <int LEN>
struct PairTree<LEN, true> {
  static constexpr int kLeaves = 1;
  template <int L0, typename Leaf>
  __device__ __forceinline__ static float eval(const Leaf &leaf) {
    return leaf.template get<L0>();
  }
};

template <int LEN>
struct PairTree<LEN, false> {
  static constexpr int kMid = ((LEN / 2 + 31) / 32) * 32;
  using Left = PairTree<kMid>;
  using Right = PairTree<LEN - kMid>;
  static constexpr int kLeaves = Left::kLeaves + Right::kLeaves;
  template <int L0, typename Leaf>
  __device__ __forceinline__ static float eval(const Leaf &leaf) {
    const float left = Left::template eval<L0>(leaf);
    return left + Right::template eval<L0 + Left::kLeaves>(leaf);
  }
};

// One leaf (at most 32 values, zero-padded): squares, then the 16-8-4-2-1 folds.
template <typename Load>
__device__ __forceinline__ float leaf_squares(const Load &load, int len) {
  float part[32];
#pragma unroll
  for (int i = 0; i < 32; i++) {
    const float v = i < len ? load(i) : 0.0f;
    part[i] = v * v;
  }
#pragma unroll
  for (int w = 16; w >= 1; w /= 2)
#pragma unroll
    for (int i = 0; i < w; i++) part[i] = part[i] + part[i + w];
  return part[0];
}

// Leaf values held by lanes: leaf L lives in lane L % 64 of register L / 64.
template <int NL>
struct LaneLeaves {
  float v[(NL + 63) / 64];
  template <int L>
  __device__ __forceinline__ float get() const {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v[L / 64]), L % 64));
  }
};

// rms_scale of one LEN-wide row, computed by a whole wave (every lane returns
// it). `at(i)` reads element i of the row (global or LDS).
template <int LEN, typename At>
__device__ __forceinline__ float rms_scale_wave(const At &at, float eps) {
  constexpr int NL = (LEN + 31) / 32;
  const int lane = threadIdx.x & 63;
  LaneLeaves<NL> leaves;
#pragma unroll
  for (int j = 0; j < (NL + 63) / 64; j++) {
    const int leaf = lane + 64 * j;
    const int len = leaf < NL ? (LEN - 32 * leaf < 32 ? LEN - 32 * leaf : 32) : 0;
    const int base = 32 * (leaf < NL ? leaf : 0);
    leaves.v[j] = leaf_squares([&](int i) { return at(base + i); }, len);
  }
  const float sum = PairTree<LEN>::template eval<0>(leaves);
  return __fdiv_rn(1.0f, __builtin_sqrtf(__fdiv_rn(sum, static_cast<float>(LEN)) + eps));
}

}  // namespace focr
