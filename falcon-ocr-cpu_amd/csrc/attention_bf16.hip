// BF16 prefill attention (the reference's `Bf16` / `Bf16Static` plans):
// kernels::attention_prefill_bf16 (src/kernels/attention/mod.rs:320-352) ->
// prefill64::bf16::compact_prefill (src/kernels/attention/prefill64/bf16.rs:
// 70-175) and its static-shift softmax (prefill64/bf16/static_shift.rs).
//
// Semantics kept from the reference: Q, K and V are rounded to BF16 (round
// to nearest even) once; QK and PV products accumulate in FP32; scores,
// maxima, denominators and outputs stay FP32; the probabilities are rounded
// to BF16 before PV. Online softmax: the denominators add the unrounded
// probabilities. Static: p = 2^(log2(e) * score) with no shift, masked keys
// +0, and the denominators add the BF16-rounded probabilities that PV uses.
// The online softmax keeps the reference's FP32 short tiles: with 32-query
// tiles and 128-key tiles as in the reference, a key tile with
// queries * keys <= 256, keys < 3 or queries < 2 (qk/pv_uses_main_path,
// prefill64.rs:65-73) is computed by reference_key_tile (prefill64.rs:
// 887-982) on the unrounded FP32 operands with the platform exp: here the
// last key tile of a 32-query wave when it is that short (fp32_tail), and
// whole rows of a last wave with one or two queries (short_rows_kernel). The
// static variant takes BF16 products everywhere, as the reference's does.
// The static softmax computes 2^t with the reference's own
// degree-3 minimax and an exact scaling by 2^n, so its probabilities round to
// the same BF16 values; the online softmax uses the hardware exp2
// (v_exp_f32, within 1e-7 of the reference's Cephes exp), its probabilities
// rounded to BF16 (2^-9 relative) right after.
//
// Layout: a pre-pass writes this call's K and V as BF16 tiles of 32 keys
// (zero past the last key) into the context scratch:
//   K: [head][tile][32 keys][8 chunks of 8 dims], chunk c of key r stored at
//      c ^ k_swizzle(r);
//   V: [kv head][tile][64 dims][4 chunks of 8 key slots], transposed, with
//      slot p = 16s + 8h + e holding key 16s + 4h + 8(e/4) + e%4 (the key
//      order in which the score registers feed the PV product), chunk c of
//      dim d stored at c ^ v_swizzle(d).
// gfx950 serves a ds_read_b128 sixteen lanes (256 bytes) at a time: the
// swizzles put the sixteen 16-byte chunks that sixteen consecutive lanes read
// (one chunk of 16 consecutive keys, or of 16 consecutive dims) in distinct
// 16-byte bank groups (also every 8 consecutive lanes within 128 bytes).
// The main kernel copies each 4 KB + 4 KB tile to LDS with the LDS-DMA path,
// double buffered, and runs v_mfma_f32_32x32x16_bf16: S^T = K Q^T (4 per
// 32-key tile), O^T += V^T P^T (4 per tile). A lane holds the 16 scores of
// one query in one half of the tile's keys, as in the FP32 kernel.
//
// Roofline: BF16 matrix cores (2.5 PFLOP/s dense) for the products; the FP32
// softmax (VALU, about 8-10 instructions per score) bounds it in practice.
// FLOPs = 4 * 64 * visible pairs per head, as for FP32.
#include "attention_split.hpp"
#include "focr_internal.hpp"

namespace focr {
namespace {

typedef float v16f __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float float2v __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(1))) const void global_void;

constexpr int kQueries = 128;   // per workgroup (4 waves x 32)
constexpr int kKeys = 32;       // per tile
constexpr int kTileBytes = 4096;  // one BF16 K or V tile
constexpr float kLog2e = 1.44269504088896340736f;

// Two FP32 values to one BF16 pair (round to nearest even): the compiler
// emits v_cvt_pk_bf16_f32 and, unlike for the same instruction written as
// inline assembly, keeps the wait state that a VALU read of a just-written
// v_exp_f32 result needs on gfx950 (without it the pair is read stale).
__device__ __forceinline__ uint32_t pack_bf16(float lo, float hi) {
  const float2v f = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f, bf16x2));
}

// exp2_lanes (bf16/static_shift.rs:277-289): n = round-to-even(t), f = t - n
// (exact), the minimax in f by FMA from the top (the reference's
// coefficients, digit for digit), times 2^n (exact while |t| < 126).
__device__ __forceinline__ float exp2_minimax(float t) {
  const float n = __builtin_rintf(t);
  const float f = t - n;
  float p = fmaf_(0.05517167f, f, 0.24261113f);
  p = fmaf_(p, f, 0.69326097f);
  p = fmaf_(p, f, 0.99992806f);
  return __builtin_ldexpf(p, static_cast<int>(n));
}

__device__ __forceinline__ int k_swizzle(int r) { return (r & 7) ^ ((r >> 3) & 1); }
__device__ __forceinline__ int v_swizzle(int d) { return ((d >> 1) & 3) ^ ((d >> 3) & 1); }

union Bf16x8 {
  bf16x8 v;
  uint4 u;
};

// ---- pre-pass: K and V to BF16 tiles ------------------------------------------
// Block (tile, head) for K: thread = (key row r, chunk c); block (tile,
// kv head) for V: thread = (dim d, chunk c).
__global__ __launch_bounds__(256) void convert_kv_kernel(const float *__restrict__ k, const float *__restrict__ v,
                                                         int total, int n_heads, int n_kv_heads, int tiles,
                                                         uint4 *__restrict__ kb, uint4 *__restrict__ vb) {
  const int tile = blockIdx.x, head = blockIdx.y;
  const int t = threadIdx.x;
  if (head < n_heads) {
    const int r = t >> 3, c = t & 7;
    const int key = tile * kKeys + r;
    uint4 out = make_uint4(0, 0, 0, 0);
    if (key < total) {
      const float4 *src = reinterpret_cast<const float4 *>(k + (static_cast<size_t>(key) * n_heads + head) * 64 + 8 * c);
      const float4 a = src[0], b = src[1];
      out = make_uint4(pack_bf16(a.x, a.y), pack_bf16(a.z, a.w), pack_bf16(b.x, b.y), pack_bf16(b.z, b.w));
    }
    kb[(static_cast<size_t>(head) * tiles + tile) * 256 + r * 8 + (c ^ k_swizzle(r))] = out;
  }
  if (head < n_kv_heads) {
    const int d = t >> 2, c = t & 3;
    float val[8];
#pragma unroll
    for (int e = 0; e < 8; e++) {
      const int p = 8 * c + e;  // slot 16s + 8h + e'
      const int s = p >> 4, hh = (p >> 3) & 1, ee = p & 7;
      const int key = tile * kKeys + 16 * s + 4 * hh + 8 * (ee >> 2) + (ee & 3);
      val[e] = key < total ? v[(static_cast<size_t>(key) * n_kv_heads + head) * 64 + d] : 0.0f;
    }
    vb[(static_cast<size_t>(head) * tiles + tile) * 256 + d * 4 + (c ^ v_swizzle(d))] =
        make_uint4(pack_bf16(val[0], val[1]), pack_bf16(val[2], val[3]), pack_bf16(val[4], val[5]),
                   pack_bf16(val[6], val[7]));
  }
}

struct Bf16Args {
  const float *q, *k, *v, *sinks;  // FP32 operands (the short tiles' path)
  const uint4 *kb, *vb;
  float *out;
  float *part;  // partial states of split query tiles (attention_split.hpp)
  int query_len, n_heads, n_kv_heads, tiles, image_start, image_end;
  int q_base, qtiles, slots;  // this launch's query tiles start at row q_base
};

// x[l % 32] op x[l % 32 + 32] in every lane (v_permlane32_swap).
__device__ __forceinline__ float halves_sum(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float halves_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  const float lo = __uint_as_float(r[0]), hi = __uint_as_float(r[1]);
  return hi > lo ? hi : lo;
}

__device__ __forceinline__ bool masked(int query, int key, const Bf16Args &a) {
  const bool image_query = query >= a.image_start && query < a.image_end;
  return key > query && !(image_query && key >= a.image_start && key < a.image_end);
}

// scale * (FMA chain over d from +0) of FP32 q and k rows (the reference's
// short-tile QK; its gemm crate order is not available, this is the chain).
__device__ __forceinline__ float score_fp32(const float *qrow, const float *krow) {
  float acc = 0.0f;
#pragma unroll
  for (int c = 0; c < 16; c++) {
    const float4 x = reinterpret_cast<const float4 *>(qrow)[c];
    const float4 y = reinterpret_cast<const float4 *>(krow)[c];
    acc = fmaf_(x.x, y.x, acc);
    acc = fmaf_(x.y, y.y, acc);
    acc = fmaf_(x.z, y.z, acc);
    acc = fmaf_(x.w, y.w, acc);
  }
  return 0.125f * acc;
}

// reference_key_tile (prefill64.rs:887-982) for keys [start, end) of the
// wave's query l32, in the online state (o, run_max, den): lane half h
// scores keys start + 2i + h, the halves trade them with v_permlane32_swap,
// and every lane then follows the keys in order: the max, p = expf(s - max),
// den += p, and acc = fma(p, v, acc) for its 32 output dims.
__device__ __forceinline__ void fp32_tail(const Bf16Args &a, int head, int kv_head, int h, int query, bool valid,
                                       bool image_query, int start, int end, v16f (&o)[2], float &run_max,
                                       float &den) {
  const float *qrow = a.q + (static_cast<size_t>(valid ? query : 0) * a.n_heads + head) * 64;
  const int pairs = (end - start + 1) / 2;
  auto pair_scores = [&](int i, float &s_even, float &s_odd) {
    const int key = start + 2 * i + h;
    float s = -__builtin_inff();
    if (key < end) {
      s = score_fp32(qrow, a.k + (static_cast<size_t>(key) * a.n_heads + head) * 64);
      const bool hidden = key > query && !(image_query && key >= a.image_start && key < a.image_end);
      s = hidden ? -__builtin_inff() : s;
    }
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(s), __float_as_uint(s), false, false);
    s_even = __uint_as_float(r[0]);  // key start + 2i (lanes 0-31)
    s_odd = __uint_as_float(r[1]);   // key start + 2i + 1 (lanes 32-63)
  };
  float block_max = -__builtin_inff();
  for (int i = 0; i < pairs; i++) {
    float se, so;
    pair_scores(i, se, so);
    block_max = __builtin_fmaxf(block_max, se);
    if (start + 2 * i + 1 < end) block_max = __builtin_fmaxf(block_max, so);
  }
  const float new_max = __builtin_fmaxf(run_max, block_max);
  if (new_max == -__builtin_inff()) return;  // every key hidden: no change
  const float rescale = run_max == -__builtin_inff() ? 0.0f : expf_acc(run_max - new_max);
#pragma unroll
  for (int d = 0; d < 2; d++)
#pragma unroll
    for (int r = 0; r < 16; r++) o[d][r] = o[d][r] * rescale;
  den = den * rescale;
  float acc[2][16];
#pragma unroll
  for (int d = 0; d < 2; d++)
#pragma unroll
    for (int r = 0; r < 16; r++) acc[d][r] = 0.0f;
  for (int i = 0; i < pairs; i++) {
    float se, so;
    pair_scores(i, se, so);
#pragma unroll
    for (int e = 0; e < 2; e++) {
      const int key = start + 2 * i + e;
      if (key >= end) break;
      const float p = expf_acc((e == 0 ? se : so) - new_max);
      den = den + p;
      const float *vrow = a.v + (static_cast<size_t>(key) * a.n_kv_heads + kv_head) * 64 + 4 * h;
#pragma unroll
      for (int d = 0; d < 2; d++)
#pragma unroll
        for (int m = 0; m < 4; m++) {
          const float4 vv = *reinterpret_cast<const float4 *>(vrow + 32 * d + 8 * m);
          acc[d][4 * m] = fmaf_(p, vv.x, acc[d][4 * m]);
          acc[d][4 * m + 1] = fmaf_(p, vv.y, acc[d][4 * m + 1]);
          acc[d][4 * m + 2] = fmaf_(p, vv.z, acc[d][4 * m + 2]);
          acc[d][4 * m + 3] = fmaf_(p, vv.w, acc[d][4 * m + 3]);
        }
    }
  }
#pragma unroll
  for (int d = 0; d < 2; d++)
#pragma unroll
    for (int r = 0; r < 16; r++) o[d][r] = o[d][r] + acc[d][r];
  run_max = new_max;
}

// Rows of a last 32-query tile that holds one or two queries: every key
// tile is short (queries * 128 <= 256), so the whole row follows
// reference_key_tile (prefill64.rs:887-982) on the FP32 operands, 128-key
// tiles in order. One workgroup per (row, head): thread t scores key t of the
// tile; thread 0 adds the probabilities in key order; thread d < 64
// accumulates output dim d over the tile's keys in order.
__global__ __launch_bounds__(128) void short_rows_kernel(Bf16Args a, int first_row, int rows) {
  __shared__ float p_tile[128];
  __shared__ float red[128];
  __shared__ float state[2];  // the new max, and the rescale factor
  const int row = first_row + blockIdx.x, head = blockIdx.y, t = threadIdx.x;
  const int kv_head = head / (a.n_heads / a.n_kv_heads);
  // tile_span of the rows' 32-query tile.
  const int last_abs = first_row + rows - 1;
  const bool intersects = first_row < a.image_end && last_abs >= a.image_start;
  const int visible_end = intersects ? (last_abs + 1 > a.image_end ? last_abs + 1 : a.image_end) : last_abs + 1;
  const float *qrow = a.q + (static_cast<size_t>(row) * a.n_heads + head) * 64;
  float run_max = -__builtin_inff(), den = 0.0f, out = 0.0f;  // out: dim t (t < 64)
  for (int start = 0; start < visible_end; start += 128) {
    const int keys = visible_end - start < 128 ? visible_end - start : 128;
    float s = -__builtin_inff();
    if (t < keys) {
      s = score_fp32(qrow, a.k + (static_cast<size_t>(start + t) * a.n_heads + head) * 64);
      s = masked(row, start + t, a) ? -__builtin_inff() : s;
    }
    red[t] = s;
    __syncthreads();
    if (t == 0) {
      float block_max = -__builtin_inff();
      for (int j = 0; j < keys; j++) block_max = __builtin_fmaxf(block_max, red[j]);
      state[0] = __builtin_fmaxf(run_max, block_max);
    }
    __syncthreads();
    const float new_max = state[0];
    if (new_max != -__builtin_inff()) {
      if (t < keys) p_tile[t] = expf_acc(s - new_max);
      const float rescale = run_max == -__builtin_inff() ? 0.0f : expf_acc(run_max - new_max);
      __syncthreads();
      den = den * rescale;
      for (int j = 0; j < keys; j++) den = den + p_tile[j];  // every thread, in key order
      if (t < 64) {
        float acc = 0.0f;
        for (int j = 0; j < keys; j++)
          acc = fmaf_(p_tile[j], a.v[(static_cast<size_t>(start + j) * a.n_kv_heads + kv_head) * 64 + t], acc);
        out = out * rescale + acc;
      }
      run_max = new_max;
    }
    __syncthreads();
  }
  if (t < 64) {
    const float lse = run_max + logf_acc(den);
    const float sink_scale = __fdiv_rn(1.0f, 1.0f + expf_acc(a.sinks[head] - lse));
    a.out[(static_cast<size_t>(row) * a.n_heads + head) * 64 + t] = __fmul_rn(__fdiv_rn(out, den), sink_scale);
  }
}

static_assert(split::kQueries == kQueries, "one query tile per split plan entry");

// A stage is two 32-key tiles (64 keys): one online-softmax update per 64
// keys, two independent score blocks in flight.
struct KvLds {
  uint4 k[2][256];  // [tile][32 keys x 8 chunks]
  uint4 v[2][256];  // [tile][64 dims x 4 chunks]
};

template <bool STATIC>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4))) void attention_bf16_kernel(Bf16Args a,
                                                                                                     split::Plan plan) {
  __shared__ KvLds buf0;
  __shared__ KvLds buf1;
  const int head = blockIdx.y;
  const int kv_head = head / (a.n_heads / a.n_kv_heads);
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int h = lane >> 5, l32 = lane & 31;
  // This workgroup's work item: a part of the query tile it.order of the plan
  // (heavy, late tiles first); parts are whole 128-key tiles of the reference.
  const split::Item it = split::find_item(plan, a.qtiles, blockIdx.x);
  const int first_query = a.q_base + (a.qtiles - 1 - it.order) * kQueries;
  const int wq0 = first_query + wave * 32;
  const int my_query = wq0 + l32;
  const bool my_valid = my_query < a.query_len;
  const bool my_image = my_query >= a.image_start && my_query < a.image_end;

  // tile_span (prefill64/span.rs:9-20) for the workgroup and for the wave.
  const int wg_queries = a.query_len - first_query < kQueries ? a.query_len - first_query : kQueries;
  const int last_abs = first_query + wg_queries - 1;
  const bool intersects = first_query < a.image_end && last_abs >= a.image_start;
  const int tile_end = intersects ? (last_abs + 1 > a.image_end ? last_abs + 1 : a.image_end) : last_abs + 1;
  const int key_begin = it.key_begin;
  const int visible_end = key_begin + it.keys < tile_end ? key_begin + it.keys : tile_end;
  const int w_queries = a.query_len - wq0 < 32 ? a.query_len - wq0 : 32;
  const int w_first = wq0, w_last = w_first + (w_queries > 0 ? w_queries : 1) - 1;
  const bool w_intersects = w_queries > 0 && w_first < a.image_end && w_last >= a.image_start;
  const int w_visible = w_queries <= 0 ? 0 : (w_intersects ? (w_last + 1 > a.image_end ? w_last + 1 : a.image_end) : w_last + 1);
  const bool w_all_image = w_first >= a.image_start && w_last < a.image_end;
  // The reference's key tiles for this 32-query tile: [128 m, min(128 (m + 1),
  // w_visible)); only the last can be short, unless the wave has at most two
  // queries (then every tile is short and short_rows_kernel takes the rows).
  const int last_tile = w_visible > 0 ? ((w_visible - 1) / 128) * 128 : 0;
  const int last_keys = w_visible - last_tile;
  const bool short_last = !STATIC && w_queries >= 3 && (w_queries * last_keys <= 256 || last_keys < 3);
  const bool short_rows = !STATIC && w_queries <= 2;
  const int w_bf16_end = short_rows ? 0 : (short_last ? last_tile : w_visible);

  // Q^T operand, step s: dims 16s + 8h .. +7 of query l32, times 1/8 (exact).
  Bf16x8 qb[4];
  {
    const float *src = a.q + (static_cast<size_t>(my_valid ? my_query : 0) * a.n_heads + head) * 64 + 8 * h;
#pragma unroll
    for (int s = 0; s < 4; s++) {
      const float4 x = reinterpret_cast<const float4 *>(src + 16 * s)[0];
      const float4 y = reinterpret_cast<const float4 *>(src + 16 * s)[1];
      const float m = my_valid ? 0.125f : 0.0f;
      qb[s].u = make_uint4(pack_bf16(m * x.x, m * x.y), pack_bf16(m * x.z, m * x.w), pack_bf16(m * y.x, m * y.y),
                           pack_bf16(m * y.z, m * y.w));
    }
  }
  v16f o[2];
#pragma unroll
  for (int d = 0; d < 2; d++)
#pragma unroll
    for (int r = 0; r < 16; r++) o[d][r] = 0.0f;
  float run_max = -__builtin_inff(), den = 0.0f;

  const uint4 *kt = a.kb + static_cast<size_t>(head) * a.tiles * 256;
  const uint4 *vt = a.vb + static_cast<size_t>(kv_head) * a.tiles * 256;
  // Each thread moves one 16-byte chunk of K and one of V per tile; wave w
  // fills bytes [1 KB w, 1 KB (w + 1)) of each. A second tile past the last
  // one repeats it (its keys are hidden by the mask: they follow every query).
  auto copy_stage = [&](KvLds &dst, int tile) {
    const int t1 = tile + 1 < a.tiles ? tile + 1 : a.tiles - 1;
    __builtin_amdgcn_global_load_lds((global_void *)(kt + static_cast<size_t>(tile) * 256 + tid),
                                     (lds_void *)(&dst.k[0][64 * wave]), 16, 0, 0);
    __builtin_amdgcn_global_load_lds((global_void *)(kt + static_cast<size_t>(t1) * 256 + tid),
                                     (lds_void *)(&dst.k[1][64 * wave]), 16, 0, 0);
    __builtin_amdgcn_global_load_lds((global_void *)(vt + static_cast<size_t>(tile) * 256 + tid),
                                     (lds_void *)(&dst.v[0][64 * wave]), 16, 0, 0);
    __builtin_amdgcn_global_load_lds((global_void *)(vt + static_cast<size_t>(t1) * 256 + tid),
                                     (lds_void *)(&dst.v[1][64 * wave]), 16, 0, 0);
  };

  auto step = [&](KvLds &cur, KvLds &next, int kstart) __attribute__((always_inline)) {
    __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0): this wave's copies of cur
    __syncthreads();                     // everyone's copies; nobody still reads next
    if (kstart + 2 * kKeys < visible_end) copy_stage(next, (kstart + 2 * kKeys) / kKeys);
    if (!(w_queries > 0 && kstart < w_bf16_end)) return;
    // S^T = K Q^T per tile t (register r: key kstart + 32 t + 8(r/4) + 4h + r%4, query l32).
    v16f st[2];
#pragma unroll
    for (int t = 0; t < 2; t++) {
      // The tile's four K fragments are read before its products.
      Bf16x8 kf[4];
#pragma unroll
      for (int s = 0; s < 4; s++) kf[s].u = cur.k[t][l32 * 8 + ((2 * s + h) ^ k_swizzle(l32))];
#pragma unroll
      for (int r = 0; r < 16; r++) st[t][r] = 0.0f;
#pragma unroll
      for (int s = 0; s < 4; s++) st[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf[s].v, qb[s].v, st[t], 0, 0, 0);
    }
    const bool full = kstart + 2 * kKeys <= w_first + 1 ||
                      (w_all_image && kstart >= a.image_start && kstart + 2 * kKeys <= a.image_end);
    if (!full) {
#pragma unroll
      for (int t = 0; t < 2; t++)
#pragma unroll
        for (int r = 0; r < 16; r++) {
          const int key = kstart + 32 * t + 8 * (r / 4) + 4 * h + (r % 4);
          const bool hidden = key > my_query && !(my_image && key >= a.image_start && key < a.image_end);
          st[t][r] = hidden ? -__builtin_inff() : st[t][r];
        }
    }
    Bf16x8 pb[2][2];
    if constexpr (STATIC) {
      // p = 2^(log2(e) * s), masked +0 (only tiles with hidden keys hold
      // -inf scores); the denominators add the rounded p a pair at a time
      // (v_dot2 of the packed pair with (1, 1)).
      float psum[2] = {0.0f, 0.0f};
      const bf16x2 ones = __builtin_bit_cast(bf16x2, 0x3F803F80u);
      auto probs = [&](bool masked) __attribute__((always_inline)) {
#pragma unroll
        for (int t = 0; t < 2; t++)
#pragma unroll
          for (int i = 0; i < 8; i++) {
            const float s0 = st[t][2 * i], s1 = st[t][2 * i + 1];
            float p0 = exp2_minimax(kLog2e * s0), p1 = exp2_minimax(kLog2e * s1);
            if (masked) {
              p0 = s0 == -__builtin_inff() ? 0.0f : p0;
              p1 = s1 == -__builtin_inff() ? 0.0f : p1;
            }
            const uint32_t pk = pack_bf16(p0, p1);
            psum[t] = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, pk), ones, psum[t], false);
            reinterpret_cast<uint32_t *>(&pb[t][i / 4].u)[i % 4] = pk;
          }
      };
      if (full)
        probs(false);
      else
        probs(true);
      den = den + halves_sum(psum[0] + psum[1]);
    } else {
      // Online step over the stage's 64 keys (softmax_pairs, bf16.rs:409-473).
      float tile_max = st[0][0];
#pragma unroll
      for (int r = 1; r < 16; r++) tile_max = __builtin_fmaxf(tile_max, st[0][r]);  // v_max3 pairs
#pragma unroll
      for (int r = 0; r < 16; r++) tile_max = __builtin_fmaxf(tile_max, st[1][r]);
      tile_max = halves_max(tile_max);
      const float new_max = tile_max > run_max ? tile_max : run_max;
      const bool skip = new_max == -__builtin_inff();
      const bool first = run_max == -__builtin_inff();
      float rescale = __builtin_amdgcn_exp2f(kLog2e * (run_max - new_max));
      rescale = first ? 0.0f : rescale;
      rescale = skip ? 1.0f : rescale;
      const float shift = skip ? 0.0f : new_max;  // skip: every s is -inf, p = +0
      // p = 2^(s log2(e) - shift log2(e)): one FMA per score (the argument
      // rounds once instead of twice; p is rounded to BF16 next).
      const float shift_l = shift * kLog2e;
      float psum[2] = {0.0f, 0.0f};
#pragma unroll
      for (int t = 0; t < 2; t++)
#pragma unroll
        for (int i = 0; i < 8; i++) {
          const float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(st[t][2 * i], kLog2e, -shift_l));
          const float p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(st[t][2 * i + 1], kLog2e, -shift_l));
          psum[t] = psum[t] + p0;
          psum[t] = psum[t] + p1;
          reinterpret_cast<uint32_t *>(&pb[t][i / 4].u)[i % 4] = pack_bf16(p0, p1);
        }
      den = den * rescale + halves_sum(psum[0] + psum[1]);
      run_max = skip ? run_max : new_max;
      if (__builtin_amdgcn_ballot_w64(rescale != 1.0f)) {
#pragma unroll
        for (int d = 0; d < 2; d++)
#pragma unroll
          for (int r = 0; r < 16; r++) o[d][r] = o[d][r] * rescale;
      }
    }
    // O^T += V^T P^T: tile t, step s takes score registers 8s .. 8s + 7
    // (keys 32 t + 16s + 4h + 8(e/4) + e%4), V^T slots 16s + 8h .. +7 of
    // dim l32 + 32d.
#pragma unroll
    for (int t = 0; t < 2; t++)
#pragma unroll
      for (int s = 0; s < 2; s++)
#pragma unroll
        for (int d = 0; d < 2; d++) {
          const int dim = l32 + 32 * d;
          Bf16x8 vf;
          vf.u = cur.v[t][dim * 4 + ((2 * s + h) ^ v_swizzle(dim))];
          o[d] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf.v, pb[t][s].v, o[d], 0, 0, 0);
        }
  };

  copy_stage(buf0, key_begin / kKeys);
  for (int kstart = key_begin; kstart < visible_end; kstart += 4 * kKeys) {
    step(buf0, buf1, kstart);
    if (kstart + 2 * kKeys < visible_end) step(buf1, buf0, kstart + 2 * kKeys);
  }

  // The short last key tile lies in one part (parts are whole 128-key tiles).
  if constexpr (!STATIC)
    if (short_last && last_tile >= key_begin && last_tile < key_begin + it.keys)
      fp32_tail(a, head, kv_head, h, my_query, my_valid, my_image, last_tile, w_visible, o, run_max, den);

  if (!my_valid || short_rows) return;
  if (it.parts > 1) {
    // A split tile: the unnormalized state, for split::merge_kernel.
    split::Args m;
    m.part = a.part;
    m.n_heads = a.n_heads;
    m.slots = a.slots;
    float *po = split::part_out(m, plan, it, head, my_query - first_query);
#pragma unroll
    for (int d = 0; d < 2; d++)
#pragma unroll
      for (int q4 = 0; q4 < 4; q4++)
        *reinterpret_cast<float4 *>(po + 32 * d + 8 * q4 + 4 * h) =
            make_float4(o[d][4 * q4], o[d][4 * q4 + 1], o[d][4 * q4 + 2], o[d][4 * q4 + 3]);
    if (h == 0) *split::part_md(m, plan, it, head, my_query - first_query) = make_float2(STATIC ? 0.0f : run_max, den);
    return;
  }

  // Normalize and apply the sink (bf16.rs:388-397, static_shift.rs:160-168).
  const float lse = STATIC ? logf_acc(den) : run_max + logf_acc(den);
  const float sink_scale = __fdiv_rn(1.0f, 1.0f + expf_acc(a.sinks[head] - lse));
  float *dst = a.out + (static_cast<size_t>(my_query) * a.n_heads + head) * 64;
#pragma unroll
  for (int d = 0; d < 2; d++)
#pragma unroll
    for (int m = 0; m < 4; m++) {
      float4 f;
      f.x = __fmul_rn(__fdiv_rn(o[d][4 * m], den), sink_scale);
      f.y = __fmul_rn(__fdiv_rn(o[d][4 * m + 1], den), sink_scale);
      f.z = __fmul_rn(__fdiv_rn(o[d][4 * m + 2], den), sink_scale);
      f.w = __fmul_rn(__fdiv_rn(o[d][4 * m + 3], den), sink_scale);
      *reinterpret_cast<float4 *>(dst + 32 * d + 8 * m + 4 * h) = f;
    }
}

}  // namespace

int launch_attention_bf16(Ctx *ctx, const float *q, const float *k, const float *v, size_t query_len,
                          size_t n_heads, size_t n_kv_heads, size_t image_start, size_t image_end,
                          const float *sinks, int softmax, float *out) {
  FOCR_REQUIRE(query_len < (size_t(1) << 30) && n_heads < 65536, FOCR_E_SHAPE, "attention shape too large");
  const size_t tiles = (query_len + kKeys - 1) / kKeys;
  const size_t k_bytes = n_heads * tiles * kTileBytes, v_bytes = n_kv_heads * tiles * kTileBytes;
  int rc = ensure_scratch(ctx, k_bytes + v_bytes);
  if (rc != FOCR_OK) return rc;
  uint4 *kb = static_cast<uint4 *>(ctx->scratch);
  uint4 *vb = reinterpret_cast<uint4 *>(static_cast<char *>(ctx->scratch) + k_bytes);
  FOCR_HIP_CHECK(hipSetDevice(ctx->device));
  hipLaunchKernelGGL(convert_kv_kernel, dim3(static_cast<unsigned>(tiles), static_cast<unsigned>(n_heads)), dim3(256),
                     0, ctx->stream, k, v, static_cast<int>(query_len), static_cast<int>(n_heads),
                     static_cast<int>(n_kv_heads), static_cast<int>(tiles), kb, vb);
  FOCR_HIP_CHECK(hipGetLastError());
  Bf16Args a;
  a.q = q;
  a.k = k;
  a.v = v;
  a.sinks = sinks;
  a.kb = kb;
  a.vb = vb;
  a.out = out;
  a.query_len = static_cast<int>(query_len);
  a.n_heads = static_cast<int>(n_heads);
  a.n_kv_heads = static_cast<int>(n_kv_heads);
  a.tiles = static_cast<int>(tiles);
  a.image_start = static_cast<int>(image_start);
  a.image_end = static_cast<int>(image_end);
  // Query rows in launches of at most split::kMaxTiles tiles, each with its
  // split plan (parts of whole 128-key tiles) and merge.
  const int short_count = softmax == FOCR_SOFTMAX_STATIC ? 0 : static_cast<int>(query_len % 32);
  const int merge_end = static_cast<int>(query_len) - (short_count == 1 || short_count == 2 ? short_count : 0);
  const size_t per_launch = static_cast<size_t>(split::kMaxTiles) * kQueries;
  for (size_t q0 = 0; q0 < query_len; q0 += per_launch) {
    const int n = static_cast<int>(query_len - q0 < per_launch ? query_len - q0 : per_launch);
    const int qtiles = (n + kQueries - 1) / kQueries;
    split::Plan plan;
    int slots = 0;
    const int items = split::make_plan(plan, qtiles, n, static_cast<int>(q0), a.image_start, a.image_end,
                                       a.n_heads, 128, split::kSplitItemsBf16, &slots);
    a.q_base = static_cast<int>(q0);
    a.qtiles = qtiles;
    a.slots = slots;
    a.part = nullptr;
    if (slots > 0) {
      const size_t part_bytes = static_cast<size_t>(slots) * n_heads * kQueries * 66 * sizeof(float);
      // The converted K/V stay at the front of the scratch; growing it would
      // discard them, so grow first and convert again.
      if (ctx->scratch_bytes < k_bytes + v_bytes + part_bytes) {
        rc = ensure_scratch(ctx, k_bytes + v_bytes + part_bytes);
        if (rc != FOCR_OK) return rc;
        kb = static_cast<uint4 *>(ctx->scratch);
        vb = reinterpret_cast<uint4 *>(static_cast<char *>(ctx->scratch) + k_bytes);
        hipLaunchKernelGGL(convert_kv_kernel, dim3(static_cast<unsigned>(tiles), static_cast<unsigned>(n_heads)),
                           dim3(256), 0, ctx->stream, k, v, static_cast<int>(query_len), static_cast<int>(n_heads),
                           static_cast<int>(n_kv_heads), static_cast<int>(tiles), kb, vb);
        FOCR_HIP_CHECK(hipGetLastError());
        a.kb = kb;
        a.vb = vb;
      }
      a.part = reinterpret_cast<float *>(static_cast<char *>(ctx->scratch) + k_bytes + v_bytes);
    }
    const dim3 grid(static_cast<unsigned>(items), static_cast<unsigned>(n_heads));
    if (softmax == FOCR_SOFTMAX_STATIC)
      hipLaunchKernelGGL(attention_bf16_kernel<true>, grid, dim3(256), 0, ctx->stream, a, plan);
    else
      hipLaunchKernelGGL(attention_bf16_kernel<false>, grid, dim3(256), 0, ctx->stream, a, plan);
    FOCR_HIP_CHECK(hipGetLastError());
    if (slots > 0) {
      split::Args m;
      m.sinks = sinks;
      m.out = out;
      m.part = a.part;
      m.query_len = static_cast<int>(query_len);
      m.n_heads = static_cast<int>(n_heads);
      m.tiles = qtiles;
      m.slots = slots;
      m.merge_end = merge_end;
      // merge_kernel's rows are relative to the launch: offset the output.
      m.out = out + q0 * n_heads * 64;
      m.merge_end = merge_end - static_cast<int>(q0);
      hipLaunchKernelGGL(split::merge_kernel, dim3(static_cast<unsigned>(qtiles), static_cast<unsigned>(n_heads), split::kMergeSplit),
                         dim3(256), 0, ctx->stream, m, plan);
      FOCR_HIP_CHECK(hipGetLastError());
    }
  }
  if (softmax != FOCR_SOFTMAX_STATIC) {
    // A last 32-query tile of one or two queries (the main kernel skips it).
    const size_t rows = query_len % 32;
    if (rows == 1 || rows == 2)
      hipLaunchKernelGGL(short_rows_kernel, dim3(static_cast<unsigned>(rows), static_cast<unsigned>(n_heads)),
                         dim3(128), 0, ctx->stream, a, static_cast<int>(query_len - rows), static_cast<int>(rows));
  }
  FOCR_HIP_CHECK(hipGetLastError());
  return FOCR_OK;
}

}  // namespace focr
