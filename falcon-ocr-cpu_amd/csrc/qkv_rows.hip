// The row step between the QKV projection and attention: split the fused QKV
// row into heads, RMS-normalize each 64-wide query and key head (unit weight,
// eps f32::EPSILON), rotate with the row's RoPE factors, and append the keys
// and values to the compact cache.
//
// Prefill rows follow fused_prefix_rows / fused_row (src/model/fused.rs:17-123):
// keys are stored for every query head (prefix keys, the GQA-expanded head
// h / (n_heads / n_kv_heads) normalized and rotated with head h's factors).
// Rows past the prefix follow split_norm_rope (src/model/rope.rs:14-86) and
// LayerCache::append's append_unique_heads (src/model/cache.rs:117-140,
// 202-216): one key per KV head, the expanded head g * repeat. Values are the
// KV heads' slices, copied. Every element sees the reference's operations:
//   scale = 1 / sqrt(sum_squares_pairwise(x) / 64 + eps)   (IEEE div, sqrt)
//   y = x * scale
//   out[2i] = y[2i] * cos - y[2i+1] * sin, out[2i+1] = y[2i] * sin + y[2i+1] * cos
// with separate roundings (no contraction), so outputs are bitwise the
// reference's.
//
// One workgroup per row (16 waves for up to 64 rows, else 4); each wave
// normalizes and rotates whole heads, lane = element, loading its heads
// (up to 32 / waves of them) before computing any. The
// 64-wide pairwise sum is two 32-leaves folded 16-8-4-2-1 (xor butterflies:
// lane i < w adds lane i + w, the other lanes' values are never read) and
// then leaf0 + leaf1 (norm_rope, decode_common.hpp).
//
// Roofline: HBM. Bytes per row = 4 * (qkv width + n_heads * 64 rope floats
// + q + keys + values written).
#include "decode_common.hpp"

namespace focr {
namespace {

struct RowArgs {
  const float *qkv, *rope;
  float *q, *prefix_k, *generated_k, *v;
  int rows, prefix_rows, n_heads, n_kv_heads;
};

using namespace decode;

// W waves per row's workgroup: 16 for a few decode rows (one or two heads a
// wave), 4 for prefill pages (enough workgroups to fill the chip anyway).
template <int W>
__global__ __launch_bounds__(64 * W) void qkv_rows_kernel(RowArgs a) {
  constexpr int kRowWaves = W;
  const int row = blockIdx.x;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int qdim = a.n_heads * 64, kdim = a.n_kv_heads * 64;
  const int repeat = a.n_heads / a.n_kv_heads;
  const float *src = a.qkv + static_cast<size_t>(row) * (qdim + 2 * kdim);
  const float2 *rope = reinterpret_cast<const float2 *>(a.rope) + static_cast<size_t>(row) * a.n_heads * 32;
  const bool prefix = row < a.prefix_rows;
  // Jobs: n_heads query heads, then the key heads (n_heads expanded ones for
  // a prefix row, n_kv_heads unique ones for a generated row). Job j reads
  // element `lane` of its source head and its rope factor pair; the first
  // kHoist jobs of a wave load before any computes, so their latencies
  // overlap (a decode row has 24 jobs, a prefill row 32).
  const int key_jobs = prefix ? a.n_heads : a.n_kv_heads;
  const int jobs = a.n_heads + key_jobs;
  auto source = [&](int job, int &x_at, int &f_at) {
    if (job < a.n_heads) {
      x_at = job * 64;
      f_at = job * 32;
    } else if (prefix) {
      const int h = job - a.n_heads;  // expanded key head: KV head h / repeat
      x_at = qdim + (h / repeat) * 64;
      f_at = h * 32;
    } else {
      const int g = job - a.n_heads;  // unique key head g = expanded head g * repeat
      x_at = qdim + g * 64;
      f_at = g * repeat * 32;
    }
  };
  auto dest = [&](int job) -> float * {
    if (job < a.n_heads) return a.q + static_cast<size_t>(row) * qdim + job * 64;
    if (prefix) return a.prefix_k + static_cast<size_t>(row) * qdim + (job - a.n_heads) * 64;
    return a.generated_k + static_cast<size_t>(row - a.prefix_rows) * kdim + (job - a.n_heads) * 64;
  };
  constexpr int kHoist = 32 / W;
  float xs[kHoist];
  float2 fs[kHoist];
#pragma unroll
  for (int i = 0; i < kHoist; i++) {
    const int job = wave + kRowWaves * i;
    if (job < jobs) {
      int x_at, f_at;
      source(job, x_at, f_at);
      xs[i] = src[x_at + lane];
      fs[i] = rope[f_at + lane / 2];
    }
  }
  // Values: the KV heads' slice of the row, copied.
  for (int i = threadIdx.x; i < kdim; i += 64 * kRowWaves)
    a.v[static_cast<size_t>(row) * kdim + i] = src[qdim + kdim + i];
#pragma unroll
  for (int i = 0; i < kHoist; i++) {
    const int job = wave + kRowWaves * i;
    if (job < jobs) dest(job)[lane] = norm_rope(xs[i], fs[i], lane);
  }
  for (int job = wave + kRowWaves * kHoist; job < jobs; job += kRowWaves) {
    int x_at, f_at;
    source(job, x_at, f_at);
    dest(job)[lane] = norm_rope(src[x_at + lane], rope[f_at + lane / 2], lane);
  }
}

}  // namespace

int launch_qkv_rows(Ctx *ctx, const float *qkv, size_t rows, const float *rope, size_t n_heads, size_t n_kv_heads,
                    size_t prefix_rows, float *q, float *prefix_k, float *generated_k, float *v) {
  FOCR_REQUIRE(rows < (size_t(1) << 31) && n_heads <= 1024, FOCR_E_SHAPE, "qkv rows: shape too large");
  RowArgs a;
  a.qkv = qkv;
  a.rope = rope;
  a.q = q;
  a.prefix_k = prefix_k;
  a.generated_k = generated_k;
  a.v = v;
  a.rows = static_cast<int>(rows);
  a.prefix_rows = static_cast<int>(prefix_rows < rows ? prefix_rows : rows);
  a.n_heads = static_cast<int>(n_heads);
  a.n_kv_heads = static_cast<int>(n_kv_heads);
  if (rows <= 64)
    hipLaunchKernelGGL(qkv_rows_kernel<16>, dim3(static_cast<unsigned>(rows)), dim3(1024), 0, ctx->stream, a);
  else
    hipLaunchKernelGGL(qkv_rows_kernel<4>, dim3(static_cast<unsigned>(rows)), dim3(256), 0, ctx->stream, a);
  FOCR_HIP_CHECK(hipGetLastError());
  return FOCR_OK;
}

}  // namespace focr
