// Decode and draft-verify attention (1..=8 query rows) over a compact KV cache,
// head_dim 64: kernels::attention_with for query_len < 4 and decode64
// (src/kernels/attention/mod.rs:256-311, online.rs:96-150, decode64.rs:22-33).
//
// The reference walks each query head's visible keys serially: 128-key tiles,
// score = dot(q, k) * (1/8), running max, rescale by exp(old - new),
// p = exp(s - max), den += p, out = fma(p, v, out), then
// out = (out / den) * 1 / (1 + exp(sink - (max + ln den))). Here the keys of
// a head are split across many waves (split-K): every wave runs that online
// softmax over its own run of keys, and a second kernel merges the
// partial states (max, denominator, unnormalized output) with the usual
// exp(m_c - M) weights before the sink step. The sums run in a different
// order than the reference's serial loop, so outputs agree within FP32
// rounding, not bitwise; exp and ln are the device libm's.
//
// Wave task = (query head h, key chunk c). Lane group lg = lane / 16 takes the
// chunk's keys 4i + lg; lane lp = lane % 16 holds dims 4lp..4lp+3 of the
// query, the key, the value and the output. Every key and value load is one
// float4 per lane (a wave instruction reads four 256-byte rows); the next 32
// keys are in flight while the current 32 are scored. Dot products reduce over the 16 lanes of a group
// with DPP (quad_perm, row_half_mirror, row_mirror: every lane ends with the
// same sum). Consecutive tasks are the query heads of one KV head on the same
// chunk, so their value rows are read together.
//
// Fused row step (launch_attention_decode_row, one generated row): the
// query is this wave's head of the new QKV row, normalized and rotated in
// the kernel (norm_rope, lane = element, then gathered to the float4 lane
// layout); the waves whose chunk holds the new position form its key and
// value the same way, use them in place of the cache's row in that one
// iteration, and the first query head of the pair writes them to the cache.
// No wave waits for another, and every value is the bits the separate row
// step would have stored, so the output is bitwise the two calls'.
//
// Roofline: HBM. Bytes per call = keys (prefix keys per query head, generated
// keys per KV head) + values per KV head over the visible keys, + q, out and
// the partial states.
#include "decode_common.hpp"

namespace focr {
namespace {

using namespace decode;

struct DecArgs {
  const float *q, *prefix_k, *generated_k, *v;
  float *part_o, *part_md;  // [rows * n_heads][chunks][64], [rows * n_heads][chunks][2]
  int prefix_len, total_len, n_heads, n_kv_heads, query_offset, image_start, image_end;
  int chunks, tasks;
  // Fused row step: the row's QKV and RoPE factors, where its query (may be
  // null), key and value go; the row is at query_offset.
  const float *qkv, *rope;
  float *q_out, *k_new, *v_new;
};

// v of lanes 4 lp .. 4 lp + 3 (lane = element to the float4 lane layout).
__device__ __forceinline__ float4 gather4(float v, int lp) {
  const int x = __float_as_int(v);
  return make_float4(__int_as_float(__builtin_amdgcn_ds_bpermute((4 * lp) << 2, x)),
                     __int_as_float(__builtin_amdgcn_ds_bpermute((4 * lp + 1) << 2, x)),
                     __int_as_float(__builtin_amdgcn_ds_bpermute((4 * lp + 2) << 2, x)),
                     __int_as_float(__builtin_amdgcn_ds_bpermute((4 * lp + 3) << 2, x)));
}

// Keys per lane group per iteration (a wave takes 4 * kKpl = 32 keys per
// iteration, double-buffered: the next iteration's keys and values are in
// flight while the current ones are scored).
constexpr int kKpl = 8;

// M: query rows. A wave task covers `iters` iterations of 32 keys. ROW: the
// fused row step (M = 1).
template <int M, bool ROW>
__global__ __launch_bounds__(256) void decode_partial_kernel(DecArgs a, int iters) {
  static_assert(!ROW || M == 1, "the fused row step takes one row");
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int lg = lane >> 4, lp = lane & 15;
  const int task = blockIdx.x * kWaves + wave;
  if (task >= a.tasks) return;
  const int repeat = a.n_heads / a.n_kv_heads;
  const int t = task % repeat, gc = task / repeat;
  const int c = gc % a.chunks, g = gc / a.chunks;
  const int h = g * repeat + t;
  const int key0 = c * iters * 4 * kKpl;

  // Geometry::visible_end per row (attention/mod.rs:60-67).
  int vis[M], limit = 0;
#pragma unroll
  for (int r = 0; r < M; r++) {
    const int abs = a.query_offset + r;
    vis[r] = abs >= a.image_start && abs < a.image_end ? a.image_end : abs + 1;
    limit = vis[r] > limit ? vis[r] : limit;
  }

  // Keys key0 + 32 it + 4 i + lg of iteration `it` (clamped to key 0 past
  // the visible keys; those are masked below).
  auto load = [&](float4 (&kb)[kKpl], float4 (&vb)[kKpl], int it) {
#pragma unroll
    for (int i = 0; i < kKpl; i++) {
      const int j = key0 + 32 * it + 4 * i + lg;
      const int jj = j < limit ? j : 0;
      const float *krow = jj < a.prefix_len
                              ? a.prefix_k + (static_cast<size_t>(jj) * a.n_heads + h) * 64
                              : a.generated_k + (static_cast<size_t>(jj - a.prefix_len) * a.n_kv_heads + g) * 64;
      kb[i] = ld4(krow + 4 * lp);
      vb[i] = ld4(a.v + (static_cast<size_t>(jj) * a.n_kv_heads + g) * 64 + 4 * lp);
    }
  };
  // Fused row step: the row's loads go first, so that waiting for them does
  // not wait for the cache reads.
  const int pos = a.query_offset;
  const bool holds = ROW && pos >= key0 && pos < key0 + iters * 4 * kKpl;  // wave-uniform
  float xq = 0.0f, xk = 0.0f;
  float2 fq = make_float2(0.0f, 0.0f), fk = fq;
  float4 vnew = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  if constexpr (ROW) {
    const int qdim = a.n_heads * 64, kdim = a.n_kv_heads * 64;
    const float2 *rope2 = reinterpret_cast<const float2 *>(a.rope);
    xq = a.qkv[h * 64 + lane];
    fq = rope2[h * 32 + lane / 2];
    if (holds) {
      // The unique key head g is the expanded head g * repeat (its factors).
      xk = a.qkv[qdim + g * 64 + lane];
      fk = rope2[g * repeat * 32 + lane / 2];
      vnew = ld4(a.qkv + qdim + kdim + g * 64 + 4 * lp);
    }
  }
  float4 ka[kKpl], va[kKpl], kb[kKpl], vb[kKpl];
  load(ka, va, 0);
  float4 qv[M];
  if constexpr (ROW) {
    const float qe = norm_rope(xq, fq, lane);
    if (a.q_out && c == 0) a.q_out[h * 64 + lane] = qe;
    qv[0] = gather4(qe, lp);
  } else {
#pragma unroll
    for (int r = 0; r < M; r++) qv[r] = ld4(a.q + (static_cast<size_t>(r) * a.n_heads + h) * 64 + 4 * lp);
  }
  // The new key of this wave's chunk: iteration it_pos, key 4 i + lg = slot.
  float4 knew = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  int it_pos = -1, slot = 0;
  if (holds) {
    const float ke = norm_rope(xk, fk, lane);
    knew = gather4(ke, lp);
    if (t == 0) {
      a.k_new[g * 64 + lane] = ke;
      if (lg == 0) *reinterpret_cast<float4 *>(a.v_new + g * 64 + 4 * lp) = vnew;
    }
    it_pos = (pos - key0) / (4 * kKpl);
    slot = (pos - key0) % (4 * kKpl);
  }
  auto patch = [&](float4 (&kk4)[kKpl], float4 (&vv4)[kKpl]) {
#pragma unroll
    for (int i = 0; i < kKpl; i++)
      if (4 * i + lg == slot) {
        kk4[i] = knew;
        vv4[i] = vnew;
      }
  };

  const float ninf = -__builtin_inff();
  float m[M], den[M];
  float4 o[M];
#pragma unroll
  for (int r = 0; r < M; r++) {
    m[r] = ninf;
    den[r] = 0.0f;
    o[r] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  }
  // Online softmax of this lane group's keys of one iteration, four at a time.
  auto consume = [&](const float4 (&kk4)[kKpl], const float4 (&vv4)[kKpl], int it) {
#pragma unroll
    for (int b = 0; b < kKpl / 4; b++) {
      float s[4][M];
#pragma unroll
      for (int kk = 0; kk < 4; kk++) {
        const int i = 4 * b + kk;
        const int j = key0 + 32 * it + 4 * i + lg;
        const float4 k = kk4[i];
#pragma unroll
        for (int r = 0; r < M; r++) {
          float d = qv[r].x * k.x;
          d = fmaf_(qv[r].y, k.y, d);
          d = fmaf_(qv[r].z, k.z, d);
          d = fmaf_(qv[r].w, k.w, d);
          d = row_sum16(d) * 0.125f;
          s[kk][r] = j < vis[r] ? d : ninf;
        }
      }
#pragma unroll
      for (int r = 0; r < M; r++) {
        float bmax = s[0][r];
#pragma unroll
        for (int kk = 1; kk < 4; kk++) bmax = s[kk][r] > bmax ? s[kk][r] : bmax;
        const float mn = bmax > m[r] ? bmax : m[r];
        if (mn == ninf) continue;
        const float rs = m[r] == ninf ? 0.0f : expf_acc(m[r] - mn);
        den[r] = den[r] * rs;
        o[r] = make_float4(o[r].x * rs, o[r].y * rs, o[r].z * rs, o[r].w * rs);
        m[r] = mn;
#pragma unroll
        for (int kk = 0; kk < 4; kk++) {
          const float p = s[kk][r] == ninf ? 0.0f : expf_acc(s[kk][r] - mn);
          const float4 v = vv4[4 * b + kk];
          den[r] = den[r] + p;
          o[r] = make_float4(fmaf_(p, v.x, o[r].x), fmaf_(p, v.y, o[r].y), fmaf_(p, v.z, o[r].z),
                             fmaf_(p, v.w, o[r].w));
        }
      }
    }
  };
  for (int it = 0; it < iters; it += 2) {
    if (it + 1 < iters) load(kb, vb, it + 1);
    if (ROW && it == it_pos) patch(ka, va);
    consume(ka, va, it);
    if (it + 1 < iters) {
      if (it + 2 < iters) load(ka, va, it + 2);
      if (ROW && it + 1 == it_pos) patch(kb, vb);
      consume(kb, vb, it + 1);
    }
  }
  // Merge the four lane groups (lanes 16 and 32 apart), then store.
#pragma unroll
  for (int r = 0; r < M; r++) {
#pragma unroll
    for (int mask = 16; mask <= 32; mask *= 2) {
      const float m2 = xor_lane(m[r], mask), d2 = xor_lane(den[r], mask);
      const float4 o2 = make_float4(xor_lane(o[r].x, mask), xor_lane(o[r].y, mask), xor_lane(o[r].z, mask),
                                    xor_lane(o[r].w, mask));
      merge(m[r], den[r], o[r], m2, d2, o2);
    }
    const size_t slot = (static_cast<size_t>(r) * a.n_heads + h) * a.chunks + c;
    if (lg == 0) *reinterpret_cast<float4 *>(a.part_o + slot * 64 + 4 * lp) = o[r];
    if (lane == 0) *reinterpret_cast<float2 *>(a.part_md + slot * 2) = make_float2(m[r], den[r]);
  }
}

template <int M, bool ROW = false>
int launch_rows(Ctx *ctx, DecArgs a, int limit, const float *sinks, float *out, size_t rows) {
  // Keys per wave: enough waves to fill the chip (about 2048), at most
  // kMaxChunks chunks per head, whole 32-key iterations.
  const long want = (static_cast<long>(limit) * a.n_heads + 2047) / 2048;
  long per_wave = ((want + 31) / 32) * 32;
  const long min_per_wave = ((static_cast<long>(limit) + kMaxChunks - 1) / kMaxChunks + 31) / 32 * 32;
  if (per_wave < min_per_wave) per_wave = min_per_wave;
  if (per_wave < 32) per_wave = 32;
  const int iters = static_cast<int>(per_wave / 32);
  a.chunks = static_cast<int>((limit + per_wave - 1) / per_wave);
  a.tasks = a.n_heads * a.chunks;
  const size_t slots = rows * static_cast<size_t>(a.n_heads) * a.chunks;
  const size_t bytes = slots * 66 * sizeof(float);
  int rc = ensure_scratch(ctx, bytes);
  if (rc != FOCR_OK) return rc;
  a.part_o = static_cast<float *>(ctx->scratch);
  a.part_md = a.part_o + slots * 64;
  const unsigned blocks = static_cast<unsigned>((a.tasks + kWaves - 1) / kWaves);
  hipLaunchKernelGGL((decode_partial_kernel<M, ROW>), dim3(blocks), dim3(64 * kWaves), 0, ctx->stream, a, iters);
  FOCR_HIP_CHECK(hipGetLastError());
  CombineArgs c;
  c.part_o = a.part_o;
  c.part_md = a.part_md;
  c.sinks = sinks;
  c.out = out;
  c.n_heads = a.n_heads;
  c.chunks = a.chunks;
  hipLaunchKernelGGL(decode_combine_kernel, dim3(static_cast<unsigned>(rows * a.n_heads)), dim3(64 * kWaves), 0,
                     ctx->stream, c);
  FOCR_HIP_CHECK(hipGetLastError());
  return FOCR_OK;
}

}  // namespace

int launch_attention_decode(Ctx *ctx, const float *q, const float *prefix_k, const float *generated_k, const float *v,
                            size_t query_len, size_t prefix_len, size_t total_len, size_t n_heads, size_t n_kv_heads,
                            size_t query_offset, size_t image_start, size_t image_end, const float *sinks,
                            float *out) {
  FOCR_REQUIRE(total_len < (size_t(1) << 30) && n_heads <= 4096, FOCR_E_SHAPE, "decode attention: shape too large");
  DecArgs a = {};
  a.q = q;
  a.prefix_k = prefix_k;
  a.generated_k = generated_k;
  a.v = v;
  a.prefix_len = static_cast<int>(prefix_len);
  a.total_len = static_cast<int>(total_len);
  a.n_heads = static_cast<int>(n_heads);
  a.n_kv_heads = static_cast<int>(n_kv_heads);
  a.query_offset = static_cast<int>(query_offset);
  a.image_start = static_cast<int>(image_start);
  a.image_end = static_cast<int>(image_end);
  // The largest visible end over the rows bounds the keys read (validated:
  // query_offset + query_len <= total_len and image_end <= prefix_len).
  size_t limit = 0;
  for (size_t r = 0; r < query_len; r++) {
    const size_t abs = query_offset + r;
    const size_t vis = abs >= image_start && abs < image_end ? image_end : abs + 1;
    limit = vis > limit ? vis : limit;
  }
  switch (query_len) {
    case 1: return launch_rows<1>(ctx, a, static_cast<int>(limit), sinks, out, query_len);
    case 2: return launch_rows<2>(ctx, a, static_cast<int>(limit), sinks, out, query_len);
    case 3: return launch_rows<3>(ctx, a, static_cast<int>(limit), sinks, out, query_len);
    case 4: return launch_rows<4>(ctx, a, static_cast<int>(limit), sinks, out, query_len);
    case 5: return launch_rows<5>(ctx, a, static_cast<int>(limit), sinks, out, query_len);
    case 6: return launch_rows<6>(ctx, a, static_cast<int>(limit), sinks, out, query_len);
    case 7: return launch_rows<7>(ctx, a, static_cast<int>(limit), sinks, out, query_len);
    case 8: return launch_rows<8>(ctx, a, static_cast<int>(limit), sinks, out, query_len);
    default: return set_error(FOCR_E_SHAPE, "decode attention takes 1..=8 query rows");
  }
}

int launch_attention_decode_row(Ctx *ctx, const float *qkv, const float *rope, const float *prefix_k, float *generated_k,
                                float *v, size_t prefix_len, size_t total_len, size_t n_heads, size_t n_kv_heads,
                                size_t image_start, size_t image_end, const float *sinks, float *q_out, float *out) {
  FOCR_REQUIRE(total_len < (size_t(1) << 30) && n_heads <= 4096, FOCR_E_SHAPE, "decode attention: shape too large");
  const size_t pos = total_len - 1, kdim = n_kv_heads * 64;
  DecArgs a = {};
  a.prefix_k = prefix_k;
  a.generated_k = generated_k;
  a.v = v;
  a.prefix_len = static_cast<int>(prefix_len);
  a.total_len = static_cast<int>(total_len);
  a.n_heads = static_cast<int>(n_heads);
  a.n_kv_heads = static_cast<int>(n_kv_heads);
  a.query_offset = static_cast<int>(pos);
  a.image_start = static_cast<int>(image_start);
  a.image_end = static_cast<int>(image_end);
  a.qkv = qkv;
  a.rope = rope;
  a.q_out = q_out;
  a.k_new = generated_k + (pos - prefix_len) * kdim;
  a.v_new = v + pos * kdim;
  // The row is past the prefix and so past the image: it sees keys 0 ..= pos.
  return launch_rows<1, true>(ctx, a, static_cast<int>(total_len), sinks, out, 1);
}

}  // namespace focr
