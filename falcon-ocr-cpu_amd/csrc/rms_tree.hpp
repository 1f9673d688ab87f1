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
// unrolls that order at compile time; a wave computes every leaf with its
// lanes (two leaves per register, the folds across lanes) and adds the leaves
// in the reference's order in straight-line code.
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

template <int CTRL>
__device__ __forceinline__ float rms_dpp(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}

// Two leaves in one register: lane i of each 32-lane half holds the square of
// element i of its leaf (zero past the row). The 16-8-4-2-1 folds
// partial[i] += partial[i + w] run across lanes: v_permlane16_swap pairs the
// two 16-lane rows of each half (w = 16); row_ror:8 pairs lanes i and i ^ 8
// (w = 8); row_ror:12, 14, 15 bring lane i + 4, i + 2, i + 1 to lane i
// (w = 4, 2, 1; only the lanes below w are used at each level). IEEE addition
// is commutative, so each sum is bitwise the reference's; lane 0 of each half
// ends with its leaf.
__device__ __forceinline__ float fold_leaf_pair(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  float s = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  s = s + rms_dpp<0x128>(s);
  s = s + rms_dpp<0x12C>(s);
  s = s + rms_dpp<0x12E>(s);
  return s + rms_dpp<0x12F>(s);
}

// Leaf L lives in lane 32 (L % 2) of register L / 2.
template <int NJ>
struct PairLeaves {
  float v[NJ];
  template <int L>
  __device__ __forceinline__ float get() const {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v[L / 2]), 32 * (L % 2)));
  }
};

// rms_scale of one LEN-wide row, computed by a whole wave (every lane returns
// it). `at(i)` reads element i of the row (global or LDS); lane l reads
// elements l, l + 64, ... (consecutive addresses across the wave), so register
// j holds leaves 2j and 2j + 1.
template <int LEN, typename At>
__device__ __forceinline__ float rms_scale_wave(const At &at, float eps) {
  constexpr int NL = (LEN + 31) / 32;
  constexpr int NJ = (NL + 1) / 2;
  const int lane = threadIdx.x & 63;
  float sq[NJ];
#pragma unroll
  for (int j = 0; j < NJ; j++) {
    const int i = 64 * j + lane;
    const float v = i < LEN ? at(i) : 0.0f;
    sq[j] = v * v;
  }
  PairLeaves<NJ> leaves;
#pragma unroll
  for (int j = 0; j < NJ; j++) leaves.v[j] = fold_leaf_pair(sq[j]);
  const float sum = PairTree<LEN>::template eval<0>(leaves);
  return __fdiv_rn(1.0f, __builtin_sqrtf(__fdiv_rn(sum, static_cast<float>(LEN)) + eps));
}

}  // namespace focr
