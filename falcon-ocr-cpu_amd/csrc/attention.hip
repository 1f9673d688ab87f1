// FP32 prefill attention with online (or static-shift) softmax over a compact
// KV cache, head_dim 64: kernels::attention_with's prefill tiles
// (src/kernels/attention/prefill64.rs:149-480, static_shift.rs:135-196).
//
// Per workgroup: one query head and 128 consecutive queries (4 waves x 32).
// Key tiles of 64 keys are staged in LDS (K for this head, V for its KV head).
// Each wave computes S^T = K Q^T with v_mfma_f32_32x32x2f32, so lane l holds
// the scores of query l % 32 (16 keys per 32-key block in each lane half):
// the running max, the denominator and the probabilities of a query stay in
// that query's two lanes, and O^T = V^T P^T takes the probabilities straight
// from the registers that hold them as the B operand. Scores are scale * dot
// with scale = 1/8, masked by the reference rule (key > query unless both are
// image tokens), softmax per query as in softmax_lanes (rescale by
// exp(old_max - new_max), p = exp(s - new_max), den = den * r + sum p), and
// the sink at the end: out = (o / den) * 1 / (1 + exp(sink - lse)).
// The matrix cores sum in their own order, so outputs match the reference
// within FP32 rounding, not bitwise.
//
// Roofline: FP32 matrix cores. FLOPs = 4 * 64 * visible (query, key) pairs
// per head (122.07 GFLOP at 6,544 tokens, 16 heads, 4,096 image tokens).
#include "focr_internal.hpp"

namespace focr {
namespace {

typedef float v16f __attribute__((ext_vector_type(16)));

constexpr int kQueries = 128;  // per workgroup (4 waves x 32)
constexpr int kKeys = 64;      // per LDS key tile
constexpr int kPitch = 64 + 4; // floats per LDS row

struct AttnArgs {
  const float *q, *prefix_k, *generated_k, *v, *sinks;
  float *out;
  int query_len, prefix_len, total_len, n_heads, n_kv_heads;
  int query_offset, image_start, image_end;
};

__device__ __forceinline__ const float *key_row(const AttnArgs &a, int position, int head) {
  if (position < a.prefix_len) return a.prefix_k + (static_cast<size_t>(position) * a.n_heads + head) * 64;
  const int repeat = a.n_heads / a.n_kv_heads;
  return a.generated_k + (static_cast<size_t>(position - a.prefix_len) * a.n_kv_heads + head / repeat) * 64;
}

template <bool STATIC, bool FAST>
__global__ __launch_bounds__(256) void attention_kernel(AttnArgs a) {
  __shared__ float ks[kKeys][kPitch];
  __shared__ float vs[kKeys][kPitch];
  const int head = blockIdx.y;
  const int kv_head = head / (a.n_heads / a.n_kv_heads);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int h = lane >> 5, l32 = lane & 31;
  const int first_query = blockIdx.x * kQueries;
  const int wq0 = first_query + wave * 32;  // this wave's first query row
  const int my_query = wq0 + l32;
  const int my_abs = a.query_offset + my_query;
  const bool my_valid = my_query < a.query_len;
  const bool my_image = my_abs >= a.image_start && my_abs < a.image_end;

  // Keys the workgroup's queries see (tile_span, prefill64/span.rs:9-20).
  const int wg_queries = a.query_len - first_query < kQueries ? a.query_len - first_query : kQueries;
  const int first_abs = a.query_offset + first_query;
  const int last_abs = first_abs + wg_queries - 1;
  const bool intersects = first_abs < a.image_end && last_abs >= a.image_start;
  const int visible_end = intersects ? (last_abs + 1 > a.image_end ? last_abs + 1 : a.image_end) : last_abs + 1;
  // This wave's own span, for skipping tiles that are masked for all its rows.
  const int w_queries = a.query_len - wq0 < 32 ? a.query_len - wq0 : 32;
  const int w_first = a.query_offset + wq0, w_last = w_first + (w_queries > 0 ? w_queries : 1) - 1;
  const bool w_intersects = w_queries > 0 && w_first < a.image_end && w_last >= a.image_start;
  const int w_visible = w_queries <= 0 ? 0 : (w_intersects ? (w_last + 1 > a.image_end ? w_last + 1 : a.image_end) : w_last + 1);

  // Q^T operand: lane holds q[my_query][32 h .. 32 h + 32).
  float qv[32];
  {
    const float *src = a.q + (static_cast<size_t>(my_valid ? my_query : 0) * a.n_heads + head) * 64 + 32 * h;
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const float4 f = reinterpret_cast<const float4 *>(src)[i];
      qv[4 * i] = my_valid ? f.x : 0.0f;
      qv[4 * i + 1] = my_valid ? f.y : 0.0f;
      qv[4 * i + 2] = my_valid ? f.z : 0.0f;
      qv[4 * i + 3] = my_valid ? f.w : 0.0f;
    }
  }
  v16f o[2];
#pragma unroll
  for (int d = 0; d < 2; d++)
#pragma unroll
    for (int r = 0; r < 16; r++) o[d][r] = 0.0f;
  float run_max = -__builtin_inff();
  float den = 0.0f;

  for (int kstart = 0; kstart < visible_end; kstart += kKeys) {
    const int keys = visible_end - kstart < kKeys ? visible_end - kstart : kKeys;
    __syncthreads();
    // Stage K (this head) and V (its KV head); rows past `keys` are zero.
    for (int idx = tid; idx < kKeys * 16; idx += 256) {
      const int r = idx >> 4, c4 = idx & 15;
      float4 kf = make_float4(0.f, 0.f, 0.f, 0.f), vf = kf;
      if (r < keys) {
        kf = reinterpret_cast<const float4 *>(key_row(a, kstart + r, head))[c4];
        vf = reinterpret_cast<const float4 *>(a.v + (static_cast<size_t>(kstart + r) * a.n_kv_heads + kv_head) * 64)[c4];
      }
      *reinterpret_cast<float4 *>(&ks[r][4 * c4]) = kf;
      *reinterpret_cast<float4 *>(&vs[r][4 * c4]) = vf;
    }
    __syncthreads();
    // Tiles that are masked for every query of the wave add nothing.
    if (w_queries <= 0 || kstart >= w_visible) continue;

    // S^T = K Q^T for two 32-key blocks; step s uses d = s + 32 h.
    v16f st[2];
#pragma unroll
    for (int kb = 0; kb < 2; kb++) {
#pragma unroll
      for (int r = 0; r < 16; r++) st[kb][r] = 0.0f;
      const float4 *krow = reinterpret_cast<const float4 *>(&ks[kb * 32 + l32][32 * h]);
#pragma unroll
      for (int i = 0; i < 8; i++) {
        const float4 kf = krow[i];
        st[kb] = __builtin_amdgcn_mfma_f32_32x32x2f32(kf.x, qv[4 * i], st[kb], 0, 0, 0);
        st[kb] = __builtin_amdgcn_mfma_f32_32x32x2f32(kf.y, qv[4 * i + 1], st[kb], 0, 0, 0);
        st[kb] = __builtin_amdgcn_mfma_f32_32x32x2f32(kf.z, qv[4 * i + 2], st[kb], 0, 0, 0);
        st[kb] = __builtin_amdgcn_mfma_f32_32x32x2f32(kf.w, qv[4 * i + 3], st[kb], 0, 0, 0);
      }
    }
    // Scale and mask. Register r of block kb holds key kb*32 + 8(r/4) + 4h + r%4.
    float tile_max = -__builtin_inff();
#pragma unroll
    for (int kb = 0; kb < 2; kb++)
#pragma unroll
      for (int r = 0; r < 16; r++) {
        const int key = kstart + kb * 32 + 8 * (r / 4) + 4 * h + (r % 4);
        float s = 0.125f * st[kb][r];
        const bool hidden = key >= kstart + keys ||
                            (key > my_abs && !(my_image && key >= a.image_start && key < a.image_end));
        s = hidden ? -__builtin_inff() : s;
        st[kb][r] = s;
        tile_max = s > tile_max ? s : tile_max;
      }
    float rescale = 1.0f;
    if constexpr (STATIC) {
      // p = exp_poly_unchecked(s), masked keys +0 (static_shift.rs:135-160).
      float psum = 0.0f;
#pragma unroll
      for (int kb = 0; kb < 2; kb++)
#pragma unroll
        for (int r = 0; r < 16; r++) {
          const float s = st[kb][r];
          const float p = s == -__builtin_inff() ? 0.0f : exp_poly_unchecked(s);
          st[kb][r] = p;
          psum = psum + p;
        }
      den = den + (psum + __shfl_xor(psum, 32));
    } else {
      // Online step (softmax_lanes, prefill64.rs:574-652) over both halves.
      const float other = __shfl_xor(tile_max, 32);
      tile_max = other > tile_max ? other : tile_max;
      const float new_max = tile_max > run_max ? tile_max : run_max;
      const bool skip = new_max == -__builtin_inff();
      const bool first = run_max == -__builtin_inff();
      rescale = FAST ? exp_poly(run_max - new_max) : expf_acc(run_max - new_max);
      rescale = first ? 0.0f : rescale;
      rescale = skip ? 1.0f : rescale;
      float psum = 0.0f;
#pragma unroll
      for (int kb = 0; kb < 2; kb++)
#pragma unroll
        for (int r = 0; r < 16; r++) {
          const float x = st[kb][r] - new_max;
          const float p = skip ? 0.0f : (FAST ? exp_poly(x) : expf_acc(x));
          st[kb][r] = p;
          psum = psum + p;
        }
      den = den * rescale + (psum + __shfl_xor(psum, 32));
      run_max = skip ? run_max : new_max;
      if (rescale != 1.0f) {
#pragma unroll
        for (int d = 0; d < 2; d++)
#pragma unroll
          for (int r = 0; r < 16; r++) o[d][r] = o[d][r] * rescale;
      }
    }
    // O^T += V^T P^T: step t of block kb uses key kb*32 + 8(t/4) + 4h + t%4.
#pragma unroll
    for (int kb = 0; kb < 2; kb++)
#pragma unroll
      for (int t = 0; t < 16; t++) {
        const int key = kb * 32 + 8 * (t / 4) + 4 * h + (t % 4);
#pragma unroll
        for (int d = 0; d < 2; d++)
          o[d] = __builtin_amdgcn_mfma_f32_32x32x2f32(vs[key][d * 32 + l32], st[kb][t], o[d], 0, 0, 0);
      }
  }
  // Normalize and apply the sink (prefill64.rs:468-479).
  const float lse = STATIC ? logf_acc(den) : run_max + logf_acc(den);
  const float sink_scale = __fdiv_rn(1.0f, 1.0f + expf_acc(a.sinks[head] - lse));
  __syncthreads();
  // Transpose through LDS: o[d][r] is output d = 32 d_blk + 8(r/4) + 4h + r%4 of
  // query l32; write rows contiguously.
  float(*stage)[kPitch] = wave < 2 ? ks + wave * 32 : vs + (wave - 2) * 32;
#pragma unroll
  for (int d = 0; d < 2; d++)
#pragma unroll
    for (int r = 0; r < 16; r++) {
      const int dim = d * 32 + 8 * (r / 4) + 4 * h + (r % 4);
      stage[l32][dim] = __fmul_rn(__fdiv_rn(o[d][r], den), sink_scale);
    }
  __syncthreads();
  for (int idx = lane; idx < 32 * 16; idx += 64) {
    const int r = idx >> 4, c4 = idx & 15;
    const int row = wq0 + r;
    if (row < a.query_len)
      reinterpret_cast<float4 *>(a.out + (static_cast<size_t>(row) * a.n_heads + head) * 64)[c4] =
          *reinterpret_cast<const float4 *>(&stage[r][4 * c4]);
  }
}

}  // namespace

int launch_attention(Ctx *ctx, const float *q, const float *prefix_k, const float *generated_k, const float *v,
                     size_t query_len, size_t prefix_len, size_t total_len, size_t n_heads, size_t n_kv_heads,
                     size_t query_offset, size_t image_start, size_t image_end, const float *sinks, int softmax,
                     int exp_mode, float *out) {
  FOCR_REQUIRE(total_len < (size_t(1) << 30) && n_heads < 65536, FOCR_E_SHAPE, "attention shape too large");
  AttnArgs a;
  a.q = q;
  a.prefix_k = prefix_k;
  a.generated_k = generated_k;
  a.v = v;
  a.sinks = sinks;
  a.out = out;
  a.query_len = static_cast<int>(query_len);
  a.prefix_len = static_cast<int>(prefix_len);
  a.total_len = static_cast<int>(total_len);
  a.n_heads = static_cast<int>(n_heads);
  a.n_kv_heads = static_cast<int>(n_kv_heads);
  a.query_offset = static_cast<int>(query_offset);
  a.image_start = static_cast<int>(image_start);
  a.image_end = static_cast<int>(image_end);
  const dim3 grid(static_cast<unsigned>((query_len + kQueries - 1) / kQueries), static_cast<unsigned>(n_heads));
  if (softmax == FOCR_SOFTMAX_STATIC)
    hipLaunchKernelGGL((attention_kernel<true, true>), grid, dim3(256), 0, ctx->stream, a);
  else if (exp_mode == FOCR_EXP_FAST)
    hipLaunchKernelGGL((attention_kernel<false, true>), grid, dim3(256), 0, ctx->stream, a);
  else
    hipLaunchKernelGGL((attention_kernel<false, false>), grid, dim3(256), 0, ctx->stream, a);
  FOCR_HIP_CHECK(hipGetLastError());
  return FOCR_OK;
}

}  // namespace focr
