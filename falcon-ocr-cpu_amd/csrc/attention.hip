// FP32 prefill attention with online (or static-shift) softmax over a compact
// KV cache, head_dim 64: kernels::attention_with's prefill tiles
// (src/kernels/attention/prefill64.rs:149-480, static_shift.rs:135-196).
//
// Per workgroup: one query head and 128 consecutive queries (4 waves x 32).
// Key tiles of 32 keys (K rows of this head, V rows of its KV head) are copied
// HBM -> LDS by the DMA path (global_load_lds, 16 bytes per lane), double
// buffered in two separate LDS arrays so the copy of tile t + 1 overlaps the
// math on tile t. A K row (256 bytes) is stored as 16 float4 chunks in the
// order c ^ (row % 16), so the 32 lanes that read one chunk of 32 different
// rows hit distinct banks; V rows are stored as they are (a lane half reads
// 32 consecutive floats of one row).
// Each wave computes S^T = K Q^T with v_mfma_f32_32x32x2f32, so lane l holds
// the scores of query l % 32 (16 keys in each lane half): the running max,
// the denominator and the probabilities of a query stay in that query's two
// lanes, and O^T = V^T P^T takes the probabilities straight from the
// registers that hold them as the B operand. Scores are scale * dot with
// scale = 1/8 (folded into Q: a power of two, so exact), masked by the
// reference rule (key > query unless both are image tokens) on the tiles
// where some key is hidden from some query of the wave, softmax per query as
// in softmax_lanes (rescale by exp(old_max - new_max), p = exp(s - new_max),
// den = den * r + sum p), and the sink at the end:
// out = (o / den) * 1 / (1 + exp(sink - lse)).
// The matrix cores sum in their own order, the online max is taken per
// 32-key tile rather than per 128 keys, and the softmax exponentials of the
// Fast and static modes are the hardware exp2 of log2(e) * x (a few ulp from
// the reference's Cephes exp_poly; ExpMode::Exact uses the device libm expf),
// so outputs match the reference within FP32 rounding, not bitwise.
//
// Roofline: FP32 matrix cores. FLOPs = 4 * 64 * visible (query, key) pairs
// per head (122.07 GFLOP at 6,544 tokens, 16 heads, 4,096 image tokens).
#include "attention_split.hpp"
#include "focr_internal.hpp"

namespace focr {
namespace {

typedef float v16f __attribute__((ext_vector_type(16)));
typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(1))) const void global_void;

constexpr int kQueries = 128;  // per workgroup (4 waves x 32)
constexpr int kKeys = 32;      // per LDS key tile

struct AttnArgs {
  const float *q, *prefix_k, *generated_k, *v, *sinks;
  float *out;
  float *part;  // partial states of split tiles (attention_split.hpp)
  int query_len, prefix_len, total_len, n_heads, n_kv_heads;
  int query_offset, image_start, image_end;
  int tiles, slots;
};
using split::kMaxTiles;
static_assert(split::kQueries == kQueries, "one query tile per split plan entry");

// One buffered key tile: [0] = K, [1] = V; 32 rows of 16 swizzled float4.
struct KvTile {
  float4 rows[2][kKeys][16];
};

__device__ __forceinline__ const float *key_row(const AttnArgs &a, int position, int head) {
  if (position < a.prefix_len) return a.prefix_k + (static_cast<size_t>(position) * a.n_heads + head) * 64;
  const int repeat = a.n_heads / a.n_kv_heads;
  return a.generated_k + (static_cast<size_t>(position - a.prefix_len) * a.n_kv_heads + head / repeat) * 64;
}

__device__ __forceinline__ int chunk(int logical, int row) { return logical ^ (row & 15); }

// x[l % 32] op x[l % 32 + 32] in every lane l (a query's two lane halves),
// with v_permlane32_swap: the first result holds the low half of x in both
// halves, the second the high half.
__device__ __forceinline__ float halves_sum(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float halves_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __builtin_fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

constexpr float kLog2e = 1.44269504088896340736f;
constexpr float kLn2 = 0.69314718055994530942f;

// The hardware exp2 (v_exp_f32, 1 ulp) of log2(e) * x: e^x within a few ulp
// of the reference's Cephes exp_poly, i.e. far inside the FP32 attention
// tolerance, at 3 instructions instead of about 17. x = -inf gives +0.
__device__ __forceinline__ float exp_hw(float x) { return __builtin_amdgcn_exp2f(kLog2e * x); }

// Copies the key tile starting at kstart into t: each wave moves rows
// 4w..4w+3 and 16+4w..16+4w+3 of K and of V, lane l -> row 4w + l / 16 (+16),
// stored chunk l % 16 (holding K chunk (l % 16) ^ (row % 16), V chunk l % 16).
// Rows at or past visible_end repeat the last visible row (in bounds); their
// scores are masked and their V rows cleared later.
__device__ __forceinline__ void copy_tile(const AttnArgs &a, KvTile &t, int kstart, int visible_end, int head,
                                          int kv_head, int wave, int lane) {
#pragma unroll
  for (int j = 0; j < 2; j++) {
    const int row = 16 * j + 4 * wave + (lane >> 4);
    const int logical = chunk(lane & 15, row);
    int pos = kstart + row;
    pos = pos < visible_end ? pos : visible_end - 1;
    const float *k_src = key_row(a, pos, head) + 4 * logical;
    const float *v_src = a.v + (static_cast<size_t>(pos) * a.n_kv_heads + kv_head) * 64 + 4 * (lane & 15);
    __builtin_amdgcn_global_load_lds((global_void *)(k_src),
                                     (lds_void *)(&t.rows[0][16 * j + 4 * wave][0]), 16, 0, 0);
    __builtin_amdgcn_global_load_lds((global_void *)(v_src),
                                     (lds_void *)(&t.rows[1][16 * j + 4 * wave][0]), 16, 0, 0);
  }
}

// Compiler-only ordering around the plain workgroup barrier: the waits are
// explicit (a __syncthreads fence would wait for every copy in flight).
__device__ __forceinline__ void plain_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

struct WaveState {
  float qv[32];  // Q^T operand, pre-scaled by 1/8: q[query][32 h + s]
  v16f o[2];     // O^T, dims 32 d + 8(r/4) + 4h + r%4 of query l32
  float run_max, den;
};

// One 32-key tile of one wave (prefill64.rs:328-480 per key tile).
template <bool STATIC, bool FAST>
__device__ __forceinline__ void tile_step(const AttnArgs &a, const KvTile &t, WaveState &w, int kstart, int keys,
                                          bool need_mask, int h, int l32, int my_abs, bool my_image) {
  // S^T = K Q^T: step s uses dims s (lanes 0-31) and 32 + s (lanes 32-63).
  v16f st;
#pragma unroll
  for (int r = 0; r < 16; r++) st[r] = 0.0f;
  // Each K chunk is read one chunk ahead of the four products that use it.
  // All eight K chunks are read before the first product (the compiler
  // would otherwise wait for each chunk right before its four products).
  float4 kall[8];
#pragma unroll
  for (int i = 0; i < 8; i++) kall[i] = t.rows[0][l32][chunk(8 * h + i, l32)];
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int i = 0; i < 8; i++) {
    const float4 kf = kall[i];
    st = __builtin_amdgcn_mfma_f32_32x32x2f32(kf.x, w.qv[4 * i], st, 0, 0, 0);
    st = __builtin_amdgcn_mfma_f32_32x32x2f32(kf.y, w.qv[4 * i + 1], st, 0, 0, 0);
    st = __builtin_amdgcn_mfma_f32_32x32x2f32(kf.z, w.qv[4 * i + 2], st, 0, 0, 0);
    st = __builtin_amdgcn_mfma_f32_32x32x2f32(kf.w, w.qv[4 * i + 3], st, 0, 0, 0);
  }
  // Register r holds key kstart + 8(r/4) + 4h + r%4.
  if (need_mask) {
#pragma unroll
    for (int r = 0; r < 16; r++) {
      const int key = kstart + 8 * (r / 4) + 4 * h + (r % 4);
      const bool hidden = key >= kstart + keys ||
                          (key > my_abs && !(my_image && key >= a.image_start && key < a.image_end));
      st[r] = hidden ? -__builtin_inff() : st[r];
    }
  }
  if constexpr (STATIC) {
    // p = exp(s) (the reference's exp_poly_unchecked), masked keys +0
    // (static_shift.rs:135-160).
    float psum = 0.0f;
#pragma unroll
    for (int r = 0; r < 16; r++) {
      const float p = exp_hw(st[r]);  // masked keys: exp(-inf) = +0
      st[r] = p;
      psum = psum + p;
    }
    w.den = w.den + halves_sum(psum);
  } else {
    // Online step (softmax_lanes, prefill64.rs:574-652) over both halves.
    float tile_max = st[0];
#pragma unroll
    for (int r = 1; r < 16; r++) tile_max = __builtin_fmaxf(tile_max, st[r]);
    tile_max = halves_max(tile_max);
    const float new_max = __builtin_fmaxf(tile_max, w.run_max);
    const bool skip = new_max == -__builtin_inff();
    const bool first = w.run_max == -__builtin_inff();
    float rescale = FAST ? exp_hw(w.run_max - new_max) : expf_acc(w.run_max - new_max);
    rescale = first ? 0.0f : rescale;
    rescale = skip ? 1.0f : rescale;
    // A skipped tile (every key hidden) has s = -inf everywhere: subtracting
    // 0 instead of -inf gives p = exp(-inf) = +0, the reference's no-op.
    const float shift = skip ? 0.0f : new_max;
    float psum = 0.0f;
#pragma unroll
    for (int r = 0; r < 16; r++) {
      const float x = st[r] - shift;
      const float p = FAST ? exp_hw(x) : expf_acc(x);
      st[r] = p;
      psum = psum + p;
    }
    w.den = w.den * rescale + halves_sum(psum);
    w.run_max = skip ? w.run_max : new_max;
    // Multiplying by 1 is exact, so the wave rescales when any lane needs it.
    if (__builtin_amdgcn_ballot_w64(rescale != 1.0f)) {
#pragma unroll
      for (int d = 0; d < 2; d++)
#pragma unroll
        for (int r = 0; r < 16; r++) w.o[d][r] = w.o[d][r] * rescale;
    }
  }
  // O^T += V^T P^T: step s uses key 8(s/4) + 4h + s%4 (the score register s);
  // the V operands are read two steps ahead of their products.
  const float *vbase = reinterpret_cast<const float *>(t.rows[1]) + 4 * h * 64 + l32;
  float v_now[2], v_next[2], v_far[2];
#pragma unroll
  for (int d = 0; d < 2; d++) {
    v_now[d] = vbase[0 * 64 + 32 * d];
    v_next[d] = vbase[1 * 64 + 32 * d];
  }
#pragma unroll
  for (int s = 0; s < 16; s++) {
    if (s + 2 < 16) {
      const int row = 8 * ((s + 2) / 4) + (s + 2) % 4;
#pragma unroll
      for (int d = 0; d < 2; d++) v_far[d] = vbase[row * 64 + 32 * d];
    }
#pragma unroll
    for (int d = 0; d < 2; d++) w.o[d] = __builtin_amdgcn_mfma_f32_32x32x2f32(v_now[d], st[s], w.o[d], 0, 0, 0);
#pragma unroll
    for (int d = 0; d < 2; d++) {
      v_now[d] = v_next[d];
      v_next[d] = v_far[d];
    }
  }
}

// Work item `item` of the plan for query head `head` on the FP32 matrix
// cores, through a ring of RING LDS key tiles (3: two tiles in flight while
// one is computed; 2: one).
template <bool STATIC, bool FAST, int RING = 3>
__device__ __forceinline__ void attention_tiles(const AttnArgs &a, const split::Plan &plan, int item, int head,
                                                KvTile &tile0, KvTile &tile1, KvTile &tile2) {
  static_assert(RING == 2 || RING == 3, "a ring of two or three tiles");
  const int kv_head = head / (a.n_heads / a.n_kv_heads);
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform
  const int h = lane >> 5, l32 = lane & 31;
  // This workgroup's work item: part `it.part` of the tile `it.order` of the
  // plan (heavy, late tiles first).
  const split::Item it = split::find_item(plan, a.tiles, item);
  const int order = it.order, part = it.part, parts = it.parts;
  const int first_query = (a.tiles - 1 - order) * kQueries;
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
  const int tile_end = intersects ? (last_abs + 1 > a.image_end ? last_abs + 1 : a.image_end) : last_abs + 1;
  // This item's keys: [key_begin, visible_end), a multiple of 32 from 0.
  const int key_begin = it.key_begin;
  const int visible_end = key_begin + it.keys < tile_end ? key_begin + it.keys : tile_end;
  // This wave's own span: tiles past it are skipped, tiles before w_first
  // (and image tiles of an all-image wave) need no mask.
  const int w_queries = a.query_len - wq0 < 32 ? a.query_len - wq0 : 32;
  const int w_first = a.query_offset + wq0, w_last = w_first + (w_queries > 0 ? w_queries : 1) - 1;
  const bool w_intersects = w_queries > 0 && w_first < a.image_end && w_last >= a.image_start;
  const int w_visible = w_queries <= 0 ? 0 : (w_intersects ? (w_last + 1 > a.image_end ? w_last + 1 : a.image_end) : w_last + 1);
  const bool w_all_image = w_first >= a.image_start && w_last < a.image_end;

  WaveState w;
  {
    const float *src = a.q + (static_cast<size_t>(my_valid ? my_query : 0) * a.n_heads + head) * 64 + 32 * h;
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const float4 f = reinterpret_cast<const float4 *>(src)[i];
      w.qv[4 * i] = my_valid ? 0.125f * f.x : 0.0f;
      w.qv[4 * i + 1] = my_valid ? 0.125f * f.y : 0.0f;
      w.qv[4 * i + 2] = my_valid ? 0.125f * f.z : 0.0f;
      w.qv[4 * i + 3] = my_valid ? 0.125f * f.w : 0.0f;
    }
  }
#pragma unroll
  for (int d = 0; d < 2; d++)
#pragma unroll
    for (int r = 0; r < 16; r++) w.o[d][r] = 0.0f;
  w.run_max = -__builtin_inff();
  w.den = 0.0f;

  // Tile t sits in array t % 3; while it is computed, tiles t + 1 and t + 2
  // are in flight. Past the last tile the copy repeats the last key into the
  // free array, so every wave always has the copies of two tiles in flight.
  auto step = [&](KvTile &cur, KvTile &ahead, int kstart) __attribute__((always_inline)) {
    const int keys = visible_end - kstart < kKeys ? visible_end - kstart : kKeys;
    // This wave's copies into cur have landed and its reads of the previous
    // tile are done; after the barrier every wave's are, so the previous
    // tile's array (ahead) is free.
    if constexpr (RING == 3)
      __builtin_amdgcn_s_waitcnt(4 | 0x0070);  // vmcnt(4) lgkmcnt(0)
    else
      __builtin_amdgcn_s_waitcnt(0x0070);  // vmcnt(0) lgkmcnt(0)
    plain_barrier();
    if (keys > 0 && keys < kKeys) {
      // Last tile: clear the V rows past the visible keys (p = 0 there, and
      // 0 * V must stay finite).
      for (int idx = tid; idx < (kKeys - keys) * 16; idx += 256)
        cur.rows[1][keys + (idx >> 4)][idx & 15] = make_float4(0.f, 0.f, 0.f, 0.f);
      __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
      plain_barrier();
    }
    const int far = kstart + (RING - 1) * kKeys;
    copy_tile(a, ahead, far < visible_end ? far : visible_end - 1, visible_end, head, kv_head, wave, lane);
    if (keys > 0 && w_queries > 0 && kstart < w_visible) {
      const bool full = keys == kKeys && (kstart + kKeys <= w_first + 1 ||
                                          (w_all_image && kstart >= a.image_start && kstart + kKeys <= a.image_end));
      tile_step<STATIC, FAST>(a, cur, w, kstart, keys, !full, h, l32, my_abs, my_image);
    }
  };
  copy_tile(a, tile0, key_begin, visible_end, head, kv_head, wave, lane);
  // Whole rounds of RING steps (a step past the last tile only waits, meets
  // the other waves and repeats a copy): the same straight-line code for
  // every round keeps the compiler's LDS-copy tracking exact, so it adds no
  // wait for the copies in flight before the reads of a landed tile.
  if constexpr (RING == 3) {
    copy_tile(a, tile1, key_begin + kKeys < visible_end ? key_begin + kKeys : visible_end - 1, visible_end, head,
              kv_head, wave, lane);
    for (int kstart = key_begin; kstart < visible_end; kstart += 3 * kKeys) {
      step(tile0, tile2, kstart);
      step(tile1, tile0, kstart + kKeys);
      step(tile2, tile1, kstart + 2 * kKeys);
    }
  } else {
    for (int kstart = key_begin; kstart < visible_end; kstart += 2 * kKeys) {
      step(tile0, tile1, kstart);
      step(tile1, tile0, kstart + kKeys);
    }
  }

  // Normalize and apply the sink (prefill64.rs:468-479); a split tile
  // stores its unnormalized state for attention_merge_kernel instead.
  const float lse = STATIC ? logf_acc(w.den) : w.run_max + logf_acc(w.den);
  const float sink_scale = __fdiv_rn(1.0f, 1.0f + expf_acc(a.sinks[head] - lse));
  const bool split = parts > 1;
  __syncthreads();
  // Transpose through LDS (8 KB per wave, swizzled like the key tiles):
  // o[d][r] is output dim 32 d + 8(r/4) + 4h + r%4 of query l32.
  float4(*stage)[16] = wave == 0 ? tile0.rows[0] : wave == 1 ? tile0.rows[1] : wave == 2 ? tile1.rows[0] : tile1.rows[1];
#pragma unroll
  for (int d = 0; d < 2; d++)
#pragma unroll
    for (int r = 0; r < 16; r++) {
      const int dim = d * 32 + 8 * (r / 4) + 4 * h + (r % 4);
      reinterpret_cast<float *>(&stage[l32][chunk(dim >> 2, l32)])[dim & 3] =
          split ? w.o[d][r] : __fmul_rn(__fdiv_rn(w.o[d][r], w.den), sink_scale);
    }
  __syncthreads();
  if (!split) {
    for (int idx = lane; idx < 32 * 16; idx += 64) {
      const int r = idx >> 4, c4 = idx & 15;
      const int row = wq0 + r;
      if (row < a.query_len)
        reinterpret_cast<float4 *>(a.out + (static_cast<size_t>(row) * a.n_heads + head) * 64)[c4] =
            stage[r][chunk(c4, r)];
    }
    return;
  }
  const size_t slot = static_cast<size_t>(plan.slot[order] + part) * a.n_heads + head;
  float *po = a.part + slot * kQueries * 64 + wave * 32 * 64;
  for (int idx = lane; idx < 32 * 16; idx += 64) {
    const int r = idx >> 4, c4 = idx & 15;
    reinterpret_cast<float4 *>(po + r * 64)[c4] = stage[r][chunk(c4, r)];
  }
  if (h == 0) {
    float *pmd = a.part + static_cast<size_t>(a.slots) * a.n_heads * kQueries * 64 + slot * kQueries * 2;
    // The static softmax has no shift: its parts merge with weight exp(0) = 1.
    reinterpret_cast<float2 *>(pmd)[wave * 32 + l32] = make_float2(STATIC ? 0.0f : w.run_max, w.den);
  }
}

template <bool STATIC, bool FAST>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3))) void attention_kernel(AttnArgs a,
                                                                                                split::Plan plan) {
  __shared__ KvTile tiles[3];
  attention_tiles<STATIC, FAST>(a, plan, blockIdx.x, blockIdx.y, tiles[0], tiles[1], tiles[2]);
}

// ---- FP32 products from FP16 pairs (focr_attention_prefill_split) --------
// The same tiles, softmax, masks, sinks and work split as attention_kernel,
// with every product of S^T = K Q^T and O^T = V^T P^T formed on
// v_mfma_f32_32x32x16_f16 from two-term FP16 expansions of power-of-two
// scaled FP32 operands: with x' = x 2^e, hi = fp16(x'), lo = fp16(x' - hi),
// so x' = hi + lo to about 2^-22 |x'|. Three products per FP32 product
// (hi.hi, hi.lo, lo.hi; lo.lo is below 2^-21 |x' y'|), FP32 accumulation and
// exact power-of-two descaling keep the result at the FP32 products' error.
// The exponents put the largest magnitude of each scale block in
// [2^14, 2^15): Q per query row (in the kernel), K per 32-key tile of a head,
// V per (KV head, dim) over every key; P by 2^14 (online softmax: P < e, the
// running maximum moving lazily) or per query by a running power-of-two
// maximum (static softmax: P = e^s), the scale folded into the exp argument
// for the hardware exp2. Per 32-key tile a wave issues 12 + 12 FP16 products (32 matrix-
// core cycles each) in place of 32 + 32 FP32 ones (64 cycles each).
// A pre-pass writes the call's K and V as two FP16 planes of 32-key tiles
// (zero past the last key), in the BF16 attention's tile layouts:
//   K: [plane][head][tile][32 keys][8 chunks of 8 dims], chunk c of key r
//      stored at c ^ ks(r);
//   V: [plane][kv head][tile][64 dims][4 chunks of 8 key slots], transposed,
//      slot 16s + 8h + e holding key 16s + 4h + 8(e/4) + e%4 (the order in
//      which the score registers feed the PV product), chunk c of dim d at
//      c ^ vs(d).
// The swizzles put the sixteen 16-byte chunks that sixteen consecutive lanes
// read in distinct bank groups.
__device__ __forceinline__ int ks(int r) { return (r & 7) ^ ((r >> 3) & 1); }
__device__ __forceinline__ int vs(int d) { return ((d >> 1) & 3) ^ ((d >> 3) & 1); }

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
union HalfFrag {
  uint4 u;
  half8 v;
};

// Eight FP32 values times 2^shift as FP16 (hi, lo) fragments (pair1).
__device__ __forceinline__ void pair8(const float (&x)[8], int shift, uint4 &hi, uint4 &lo) {
  uint16_t h[8], l[8];
#pragma unroll
  for (int e = 0; e < 8; e++) pair1(x[e], shift, h[e], l[e]);
  hi = make_uint4(h[0] | h[1] << 16, h[2] | h[3] << 16, h[4] | h[5] << 16, h[6] | h[7] << 16);
  lo = make_uint4(l[0] | l[1] << 16, l[2] | l[3] << 16, l[4] | l[5] << 16, l[6] | l[7] << 16);
}

// Per (KV head, dim): the largest finite |v| over every key, as float bits
// (atomic unsigned max of non-negative floats). Block (KV head, 128 keys):
// thread = dims 4 d4 .. 4 d4 + 3 (d4 = t % 16) of keys kq, kq + 16, ...
// (kq = t / 16): eight 16-byte loads in flight, sixteen threads per 256-byte
// row; one atomic per dim and block. (A block per 32-key tile made four
// times the atomics per address, 510 at 16,320 keys, and took 25 us there.)
__global__ __launch_bounds__(256) void pair_vmax_kernel(const float *__restrict__ v, int total, int n_kv_heads,
                                                        unsigned *__restrict__ vmax, unsigned *__restrict__ nonfinite) {
  __shared__ float part[16][65];
  const int head = blockIdx.x, t = threadIdx.x;
  const int d4 = t & 15, kq = t >> 4;
  const int k0 = blockIdx.y * 128;
  float4 x[8];
#pragma unroll
  for (int j = 0; j < 8; j++) {
    const int key = k0 + kq + 16 * j;
    x[j] = key < total ? *reinterpret_cast<const float4 *>(v + (static_cast<size_t>(key) * n_kv_heads + head) * 64 + 4 * d4)
                       : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  }
  float m[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  bool bad = false;
#pragma unroll
  for (int j = 0; j < 8; j++) {
    m[0] = __builtin_fmaxf(m[0], finite_abs(x[j].x));
    m[1] = __builtin_fmaxf(m[1], finite_abs(x[j].y));
    m[2] = __builtin_fmaxf(m[2], finite_abs(x[j].z));
    m[3] = __builtin_fmaxf(m[3], finite_abs(x[j].w));
    bad = bad || !is_finite(x[j].x) || !is_finite(x[j].y) || !is_finite(x[j].z) || !is_finite(x[j].w);
  }
  if (bad) atomicOr(nonfinite, 1u);
#pragma unroll
  for (int e = 0; e < 4; e++) part[kq][4 * d4 + e] = m[e];
  __syncthreads();
  if (t < 64) {
    float r = part[0][t];
#pragma unroll
    for (int i = 1; i < 16; i++) r = __builtin_fmaxf(r, part[i][t]);
    atomicMax(vmax + head * 64 + t, __float_as_uint(r));
  }
}

__global__ __launch_bounds__(64) void pair_zero_kernel(unsigned *__restrict__ p, int n) {
  const int i = blockIdx.x * 64 + threadIdx.x;
  if (i < n) p[i] = 0u;
}

// Block (tile, head): K of query head `head` (thread = key row r, chunk c;
// the tile's exponent from the block's largest magnitude, kexp[head][tile])
// and, for head < n_kv_heads, V of that KV head (thread = dim d, chunk c;
// the dim's exponent from vmax).
__global__ __launch_bounds__(256) void pair_kv_kernel(const float *__restrict__ k, const float *__restrict__ v,
                                                      int total, int n_heads, int n_kv_heads, int tiles,
                                                      const unsigned *__restrict__ vmax, uint4 *__restrict__ kp,
                                                      uint4 *__restrict__ vp, int *__restrict__ kexp,
                                                      unsigned *__restrict__ nonfinite) {
  __shared__ float wmax[4];
  const int tile = blockIdx.x, head = blockIdx.y, t = threadIdx.x;
  const size_t kplane = static_cast<size_t>(n_heads) * tiles * 256, vplane = static_cast<size_t>(n_kv_heads) * tiles * 256;
  {
    const int r = t >> 3, c = t & 7;
    const int key = tile * kKeys + r;
    float val[8];
#pragma unroll
    for (int e = 0; e < 8; e++) val[e] = 0.0f;
    if (key < total) {
      const float4 *src = reinterpret_cast<const float4 *>(k + (static_cast<size_t>(key) * n_heads + head) * 64 + 8 * c);
      const float4 x = src[0], y = src[1];
      val[0] = x.x; val[1] = x.y; val[2] = x.z; val[3] = x.w;
      val[4] = y.x; val[5] = y.y; val[6] = y.z; val[7] = y.w;
    }
    float m = 0.0f;
    bool bad = false;
#pragma unroll
    for (int e = 0; e < 8; e++) {
      m = __builtin_fmaxf(m, finite_abs(val[e]));
      bad = bad || !is_finite(val[e]);
    }
    if (bad) atomicOr(nonfinite, 1u);
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) m = __builtin_fmaxf(m, __shfl_xor(m, off));
    if ((t & 63) == 0) wmax[t >> 6] = m;
    __syncthreads();
    const int ex = pair_exp(__builtin_fmaxf(__builtin_fmaxf(wmax[0], wmax[1]), __builtin_fmaxf(wmax[2], wmax[3])));
    if (t == 0) kexp[head * tiles + tile] = ex;
    uint4 hi, lo;
    pair8(val, 15 - ex, hi, lo);
    const size_t i = (static_cast<size_t>(head) * tiles + tile) * 256 + r * 8 + (c ^ ks(r));
    kp[i] = hi;
    kp[kplane + i] = lo;
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
    uint4 hi, lo;
    pair8(val, 15 - pair_exp(__uint_as_float(vmax[head * 64 + d])), hi, lo);
    const size_t i = (static_cast<size_t>(head) * tiles + tile) * 256 + d * 4 + (c ^ vs(d));
    vp[i] = hi;
    vp[vplane + i] = lo;
  }
}

// One buffered key tile of the pair kernel: [plane][256 chunks] of K and V.
struct PairKvTile {
  uint4 k[2][256];
  uint4 v[2][256];
};

// Copies pair tile `kt` (this head's K planes, its KV head's V planes) into
// t: thread tid moves chunk tid of each of the four 4 KB planes.
__device__ __forceinline__ void copy_pair_tile(PairKvTile &t, const uint4 *kp, const uint4 *vp, size_t kplane,
                                               size_t vplane, int tiles, int kt, int head, int kv_head, int wave,
                                               int tid) {
#pragma unroll
  for (int p = 0; p < 2; p++) {
    __builtin_amdgcn_global_load_lds((global_void *)(kp + p * kplane + (static_cast<size_t>(head) * tiles + kt) * 256 + tid),
                                     (lds_void *)(&t.k[p][64 * wave]), 16, 0, 0);
    __builtin_amdgcn_global_load_lds((global_void *)(vp + p * vplane + (static_cast<size_t>(kv_head) * tiles + kt) * 256 + tid),
                                     (lds_void *)(&t.v[p][64 * wave]), 16, 0, 0);
  }
}

// Two FP32 values as an FP16 pair each, rounded toward zero: hi of both in
// one word, lo of both in the other (x >= 0 here, so lo >= 0 and
// x = hi + lo to 2^-21 |x|).
__device__ __forceinline__ void pair2_rtz(float x0, float x1, uint32_t &hi, uint32_t &lo) {
  const auto h = __builtin_amdgcn_cvt_pkrtz(x0, x1);
  const auto l = __builtin_amdgcn_cvt_pkrtz(x0 - static_cast<float>(h[0]), x1 - static_cast<float>(h[1]));
  hi = __builtin_bit_cast(uint32_t, h);
  lo = __builtin_bit_cast(uint32_t, l);
}

// How far the online softmax lets a tile's scores exceed the running maximum
// before it moves the maximum: 2^14 e^1 = 44,536 < 65,504, the FP16 range.
constexpr float kLazyMax = 1.0f;

// One 32-key tile of one wave: tile_step's softmax with FP16-pair products.
// c = the score factor (the Q, K and 1/8 descale, times log2(e) for the
// static form's base-2 exp); pexp = the static form's running P exponent.
template <bool STATIC, bool FAST>
__device__ __forceinline__ void pair_tile_step(const PairKvTile &t, const HalfFrag (&qf)[2][4], v16f (&o)[2],
                                               float &run_max, float &den, int &pexp, float c, int kstart, int keys,
                                               bool need_mask, int h, int l32, int my_abs, bool my_image,
                                               int image_start, int image_end) {
  // S^T = K Q^T: step s covers dims 16 s .. 16 s + 15 (lane half h: 8 h ..);
  // products (lo, hi), (hi, lo), (hi, hi).
  // Fragments are read step by step (the registers hold four waves per SIMD).
  constexpr int pa[3] = {1, 0, 0}, pb[3] = {0, 1, 0};
  v16f st;
#pragma unroll
  for (int r = 0; r < 16; r++) st[r] = 0.0f;
#pragma unroll
  for (int s = 0; s < 4; s++) {
    HalfFrag kf[2];
#pragma unroll
    for (int p = 0; p < 2; p++) kf[p].u = t.k[p][l32 * 8 + ((2 * s + h) ^ ks(l32))];
#pragma unroll
    for (int q = 0; q < 3; q++) st = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf[pa[q]].v, qf[pb[q]][s].v, st, 0, 0, 0);
  }
  // Register r holds key kstart + 8(r/4) + 4h + r%4. The descale c (> 0) is
  // exact, a power of two, times log2(e) for the hardware exp2 (one rounding,
  // as exp_hw's log2(e) * s). It is applied inside the max and the exp
  // argument: c max(st) = max(c st), and fma(st, c, k) rounds c st + k once.
  if (need_mask) {
#pragma unroll
    for (int r = 0; r < 16; r++) {
      const int key = kstart + 8 * (r / 4) + 4 * h + (r % 4);
      const bool hidden = key >= kstart + keys || (key > my_abs && !(my_image && key >= image_start && key < image_end));
      st[r] = hidden ? -__builtin_inff() : st[r];
    }
  }
  // P enters its FP16 pair scaled by a power of two: the static form and the
  // online form with the hardware exp fold it into the exp argument (an
  // integer added inside the argument's one rounding, their c holding
  // log2(e)); the online form with the platform exp scales P by 2^14 after.
  int shift = 0;
  if constexpr (STATIC) {
    // The tile's largest P (exp2 is monotonic) moves the running exponent
    // before any P is formed; the output follows it by exact powers of two.
    float tmax = st[0];
#pragma unroll
    for (int r = 1; r < 16; r++) tmax = __builtin_fmaxf(tmax, st[r]);
    const int e = pair_exp(__builtin_amdgcn_exp2f(halves_max(tmax) * c));  // masked keys: +0
    if (__builtin_amdgcn_ballot_w64(e > pexp)) {
      const float f = __builtin_ldexpf(1.0f, pexp - e);
      const bool up = e > pexp;
#pragma unroll
      for (int d = 0; d < 2; d++)
#pragma unroll
        for (int r = 0; r < 16; r++) o[d][r] = up ? o[d][r] * f : o[d][r];
      pexp = up ? e : pexp;
    }
    // P' = 2^(15 - pexp) P <= 2^15; the denominator adds the unscaled P.
    const float fs = static_cast<float>(15 - pexp);
    float ps[16];
#pragma unroll
    for (int r = 0; r < 16; r++) {
      const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(st[r], c, fs));
      st[r] = p;
      ps[r] = p;
    }
#pragma unroll
    for (int w = 1; w < 16; w *= 2)
#pragma unroll
      for (int r = 0; r < 16; r += 2 * w) ps[r] = ps[r] + ps[r + w];
    den = den + __builtin_ldexpf(halves_sum(ps[0]), pexp - 15);
  } else {
    // Scores, maximum and the lazy threshold in log2 units with the hardware
    // exp (FAST), natural units with the platform exp.
    constexpr float lazy = FAST ? kLazyMax * kLog2e : kLazyMax;
    float tile_max = st[0];
#pragma unroll
    for (int r = 1; r < 16; r++) tile_max = __builtin_fmaxf(tile_max, st[r]);
    tile_max = halves_max(tile_max) * c;
    // The running maximum moves only when the tile's exceeds it by more than
    // kLazyMax (and at the first visible key): P = e^(s - max) then stays
    // below e^kLazyMax, 2^14 P inside the FP16 range, and most tiles leave the
    // output unscaled. Output and denominator always share the maximum, so
    // their ratio is the softmax's.
    const bool raise = tile_max > run_max + lazy;
    const float new_max = raise ? tile_max : run_max;
    const bool skip = new_max == -__builtin_inff();
    const bool first = run_max == -__builtin_inff();
    float rescale = FAST ? __builtin_amdgcn_exp2f(run_max - new_max) : expf_acc(run_max - new_max);
    rescale = first ? 0.0f : rescale;
    rescale = raise ? rescale : 1.0f;
    const float shift_max = skip ? 0.0f : new_max;
    const float off = FAST ? 14.0f - shift_max : -shift_max;  // FAST: P' = 2^14 P < 2^14 e
    float ps[16];
#pragma unroll
    for (int r = 0; r < 16; r++) {
      const float x = __builtin_fmaf(st[r], c, off);
      const float p = FAST ? __builtin_amdgcn_exp2f(x) : expf_acc(x);
      st[r] = p;
      ps[r] = p;
    }
    // The tile's sum as a pairwise tree (depth 4 instead of a 16-long chain).
#pragma unroll
    for (int w = 1; w < 16; w *= 2)
#pragma unroll
      for (int r = 0; r < 16; r += 2 * w) ps[r] = ps[r] + ps[r + w];
    const float tsum = halves_sum(ps[0]);
    den = den * rescale + (FAST ? __builtin_ldexpf(tsum, -14) : tsum);
    run_max = skip ? run_max : new_max;
    if (__builtin_amdgcn_ballot_w64(rescale != 1.0f)) {
#pragma unroll
      for (int d = 0; d < 2; d++)
#pragma unroll
        for (int r = 0; r < 16; r++) o[d][r] = o[d][r] * rescale;
    }
    if constexpr (!FAST) shift = 14;  // P < e^kLazyMax
  }
  // O^T += V^T P^T: step s2 takes score registers 8 s2 .. 8 s2 + 7 (keys
  // 16 s2 + 4h + 8(e/4) + e%4) as the B operand, V^T slots 16 s2 + 8h .. of
  // dim l32 + 32 d as the A operand; products (lo, hi), (hi, lo), (hi, hi).
#pragma unroll
  for (int s2 = 0; s2 < 2; s2++) {
    HalfFrag pf[2];
    {
      uint32_t hw[4], lw[4];
#pragma unroll
      for (int e = 0; e < 4; e++)
        pair2_rtz(shift ? __builtin_ldexpf(st[8 * s2 + 2 * e], shift) : st[8 * s2 + 2 * e],
                  shift ? __builtin_ldexpf(st[8 * s2 + 2 * e + 1], shift) : st[8 * s2 + 2 * e + 1], hw[e], lw[e]);
      pf[0].u = make_uint4(hw[0], hw[1], hw[2], hw[3]);
      pf[1].u = make_uint4(lw[0], lw[1], lw[2], lw[3]);
    }
    HalfFrag vf[2][2];
#pragma unroll
    for (int p = 0; p < 2; p++)
#pragma unroll
      for (int d = 0; d < 2; d++) {
        const int dim = l32 + 32 * d;
        vf[p][d].u = t.v[p][dim * 4 + ((2 * s2 + h) ^ vs(dim))];
      }
#pragma unroll
    for (int q = 0; q < 3; q++)
#pragma unroll
      for (int d = 0; d < 2; d++)
        o[d] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf[pa[q]][d].v, pf[pb[q]].v, o[d], 0, 0, 0);
  }
}

// Pure prefill only (every key a prefix key, queries = keys from position 0).
template <bool STATIC, bool FAST>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4))) void attention_pair_kernel(
    AttnArgs a, const uint4 *__restrict__ kp, const uint4 *__restrict__ vp, const int *__restrict__ kexp,
    const unsigned *__restrict__ vmax, const unsigned *__restrict__ nonfinite, size_t kplane, size_t vplane,
    int ktiles, split::Plan plan) {
  static_assert(sizeof(PairKvTile) == sizeof(KvTile), "the two bodies' key tiles share the LDS");
  __shared__ union {
    PairKvTile pair[2];
    KvTile f32[2];
  } lds;
  __shared__ int vexp[64];
  if (*nonfinite != 0u) {
    // The pre-pass found a non-finite K or V value: an infinity in an FP16
    // pair meets zero halves (0 * inf = NaN) where FP32 products give +-inf
    // (a -inf score is a zero probability), so the whole call takes the FP32
    // products (attention_kernel's body on a ring of two tiles), with the
    // same plan and partial-state layout. Its registers spill under this
    // kernel's budget; it runs only for such calls.
    attention_tiles<STATIC, FAST, 2>(a, plan, blockIdx.x, blockIdx.y, lds.f32[0], lds.f32[1], lds.f32[1]);
    return;
  }
  PairKvTile &tile0 = lds.pair[0];
  PairKvTile &tile1 = lds.pair[1];
  const int head = blockIdx.y;
  const int kv_head = head / (a.n_heads / a.n_kv_heads);
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int h = lane >> 5, l32 = lane & 31;
  const split::Item it = split::find_item(plan, a.tiles, blockIdx.x);
  const int order = it.order, part = it.part, parts = it.parts;
  const int first_query = (a.tiles - 1 - order) * kQueries;
  const int wq0 = first_query + wave * 32;
  const int my_query = wq0 + l32;
  const int my_abs = a.query_offset + my_query;
  const bool my_valid = my_query < a.query_len;
  const bool my_image = my_abs >= a.image_start && my_abs < a.image_end;
  const int wg_queries = a.query_len - first_query < kQueries ? a.query_len - first_query : kQueries;
  const int first_abs = a.query_offset + first_query;
  const int last_abs = first_abs + wg_queries - 1;
  const bool intersects = first_abs < a.image_end && last_abs >= a.image_start;
  const int tile_end = intersects ? (last_abs + 1 > a.image_end ? last_abs + 1 : a.image_end) : last_abs + 1;
  const int key_begin = it.key_begin;
  const int visible_end = key_begin + it.keys < tile_end ? key_begin + it.keys : tile_end;
  const int w_queries = a.query_len - wq0 < 32 ? a.query_len - wq0 : 32;
  const int w_first = a.query_offset + wq0, w_last = w_first + (w_queries > 0 ? w_queries : 1) - 1;
  const bool w_intersects = w_queries > 0 && w_first < a.image_end && w_last >= a.image_start;
  const int w_visible = w_queries <= 0 ? 0 : (w_intersects ? (w_last + 1 > a.image_end ? w_last + 1 : a.image_end) : w_last + 1);
  const bool w_all_image = w_first >= a.image_start && w_last < a.image_end;

  // Q^T operand, step s: dims 16 s + 8 h .. + 7 of query l32, scaled by the
  // row's exponent (both lane halves of a query agree on it).
  HalfFrag qf[2][4];
  int qexp;
  {
    const float *src = a.q + (static_cast<size_t>(my_valid ? my_query : 0) * a.n_heads + head) * 64 + 8 * h;
    float qv[4][8];
    float m = 0.0f;
#pragma unroll
    for (int s = 0; s < 4; s++) {
      const float4 x = reinterpret_cast<const float4 *>(src + 16 * s)[0];
      const float4 y = reinterpret_cast<const float4 *>(src + 16 * s)[1];
      const float z = my_valid ? 1.0f : 0.0f;
      qv[s][0] = z * x.x; qv[s][1] = z * x.y; qv[s][2] = z * x.z; qv[s][3] = z * x.w;
      qv[s][4] = z * y.x; qv[s][5] = z * y.y; qv[s][6] = z * y.z; qv[s][7] = z * y.w;
#pragma unroll
      for (int e = 0; e < 8; e++) m = __builtin_fmaxf(m, finite_abs(qv[s][e]));
    }
    qexp = pair_exp(halves_max(m));
#pragma unroll
    for (int s = 0; s < 4; s++) pair8(qv[s], 15 - qexp, qf[0][s].u, qf[1][s].u);
  }
  // The score factor of a key tile with exponent ke: 2^(qexp + ke - 30) / 8,
  // times log2(e) for the static form.
  const float cbase = STATIC || FAST ? kLog2e : 1.0f;  // log2 units for the hardware exp2
  v16f o[2];
#pragma unroll
  for (int d = 0; d < 2; d++)
#pragma unroll
    for (int r = 0; r < 16; r++) o[d][r] = 0.0f;
  float run_max = -__builtin_inff(), den = 0.0f;
  int pexp = kPairMinExp;

  // Tile t sits in array t % 2; tile t + 1 is in flight while it is computed
  // (past the last tile the copy repeats the last one). Two arrays (32 KB)
  // and at most 128 VGPRs keep four waves per SIMD.
  auto step = [&](PairKvTile &cur, PairKvTile &ahead, int kstart) __attribute__((always_inline)) {
    const int keys = visible_end - kstart < kKeys ? visible_end - kstart : kKeys;
    __builtin_amdgcn_s_waitcnt(0x0070);  // vmcnt(0) lgkmcnt(0): this tile's four copies
    plain_barrier();
    if (keys > 0 && keys < kKeys) {
      // Last tile: clear the V slots of keys past the visible ones in both
      // planes (p = 0 there, and 0 * V must stay finite).
      for (int idx = tid; idx < 2 * 64 * 32; idx += 256) {
        const int p = idx >> 11, rem = idx & 2047, dim = rem >> 5, slot = rem & 31;
        const int s2 = slot >> 4, hh = (slot >> 3) & 1, e = slot & 7;
        const int key = 16 * s2 + 4 * hh + 8 * (e >> 2) + (e & 3);
        if (key >= keys)
          reinterpret_cast<uint16_t *>(&cur.v[p][dim * 4 + ((slot >> 3) ^ vs(dim))])[e] = 0;
      }
      __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
      plain_barrier();
    }
    const int next = kstart + kKeys;
    copy_pair_tile(ahead, kp, vp, kplane, vplane, ktiles, (next < visible_end ? next : visible_end - 1) / kKeys, head,
                   kv_head, wave, tid);
    if (keys > 0 && w_queries > 0 && kstart < w_visible) {
      const bool full = keys == kKeys && (kstart + kKeys <= w_first + 1 ||
                                          (w_all_image && kstart >= a.image_start && kstart + kKeys <= a.image_end));
      const int ke = kexp[head * ktiles + kstart / kKeys];
      // Kept a normal float (> 0): it is clamped only where every scaled
      // score (|q'.k'| < 64 2^30) times the true factor is below 2^-89, so
      // exp gives 1 with either factor.
      const float c = __builtin_fmaxf(__builtin_ldexpf(cbase, qexp + ke - 33), 1.17549435e-38f);
      pair_tile_step<STATIC, FAST>(cur, qf, o, run_max, den, pexp, c, kstart, keys, !full, h, l32, my_abs, my_image,
                                   a.image_start, a.image_end);
    }
  };
  copy_pair_tile(tile0, kp, vp, kplane, vplane, ktiles, key_begin / kKeys, head, kv_head, wave, tid);
  for (int kstart = key_begin; kstart < visible_end; kstart += 2 * kKeys) {
    step(tile0, tile1, kstart);
    step(tile1, tile0, kstart + kKeys);
  }

  // The running maximum in natural units (FAST keeps it in log2 units).
  const float nat_max = FAST ? run_max * kLn2 : run_max;
  const float lse = STATIC ? logf_acc(den) : nat_max + logf_acc(den);
  const float sink_scale = __fdiv_rn(1.0f, 1.0f + expf_acc(a.sinks[head] - lse));
  const bool split = parts > 1;
  const int pshift = STATIC ? 15 - pexp : 14;
  if (tid < 64) vexp[tid] = pair_exp(__uint_as_float(vmax[kv_head * 64 + tid]));
  // The copies still in flight must land before the arrays are reused.
  __builtin_amdgcn_s_waitcnt(0x0070);  // vmcnt(0) lgkmcnt(0)
  __syncthreads();
  // Transpose through LDS (8 KB per wave): o[d][r] is output dim
  // 32 d + 8(r/4) + 4h + r%4 of query l32, times 2^(pshift + 15 - e_dim).
  float4(*stage)[16] = reinterpret_cast<float4(*)[16]>(
      wave == 0 ? &tile0.k[0][0] : wave == 1 ? &tile0.v[0][0] : wave == 2 ? &tile1.k[0][0] : &tile1.v[0][0]);
#pragma unroll
  for (int d = 0; d < 2; d++)
#pragma unroll
    for (int r = 0; r < 16; r++) {
      const int dim = d * 32 + 8 * (r / 4) + 4 * h + (r % 4);
      const float ov = __builtin_ldexpf(o[d][r], vexp[dim] - 15 - pshift);
      reinterpret_cast<float *>(&stage[l32][chunk(dim >> 2, l32)])[dim & 3] =
          split ? ov : __fmul_rn(__fdiv_rn(ov, den), sink_scale);
    }
  __syncthreads();
  if (!split) {
    for (int idx = lane; idx < 32 * 16; idx += 64) {
      const int r = idx >> 4, c4 = idx & 15;
      const int row = wq0 + r;
      if (row < a.query_len)
        reinterpret_cast<float4 *>(a.out + (static_cast<size_t>(row) * a.n_heads + head) * 64)[c4] =
            stage[r][chunk(c4, r)];
    }
    return;
  }
  const size_t slot = static_cast<size_t>(plan.slot[order] + part) * a.n_heads + head;
  float *po = a.part + slot * kQueries * 64 + wave * 32 * 64;
  for (int idx = lane; idx < 32 * 16; idx += 64) {
    const int r = idx >> 4, c4 = idx & 15;
    reinterpret_cast<float4 *>(po + r * 64)[c4] = stage[r][chunk(c4, r)];
  }
  if (h == 0) {
    float *pmd = a.part + static_cast<size_t>(a.slots) * a.n_heads * kQueries * 64 + slot * kQueries * 2;
    reinterpret_cast<float2 *>(pmd)[wave * 32 + l32] = make_float2(STATIC ? 0.0f : nat_max, den);
  }
}

}  // namespace

namespace {

// One launch (plus the merge) for at most kMaxTiles query tiles.
int launch_tiles(Ctx *ctx, AttnArgs a, int softmax, int exp_mode) {
  // Split plan (attention_split.hpp): parts of whole 32-key tiles.
  const int tiles = (a.query_len + kQueries - 1) / kQueries;
  split::Plan plan;
  int slots = 0;
  const int items = split::make_plan(plan, tiles, a.query_len, a.query_offset, a.image_start, a.image_end, a.n_heads,
                                     kKeys, split::kSplitItemsF32, &slots);
  a.tiles = tiles;
  a.slots = slots;
  a.part = nullptr;
  if (slots > 0) {
    const size_t bytes = static_cast<size_t>(slots) * a.n_heads * kQueries * 66 * sizeof(float);
    int rc = ensure_scratch(ctx, bytes);
    if (rc != FOCR_OK) return rc;
    a.part = static_cast<float *>(ctx->scratch);
  }
  const dim3 grid(static_cast<unsigned>(items), static_cast<unsigned>(a.n_heads));
  if (softmax == FOCR_SOFTMAX_STATIC)
    hipLaunchKernelGGL((attention_kernel<true, true>), grid, dim3(256), 0, ctx->stream, a, plan);
  else if (exp_mode == FOCR_EXP_FAST)
    hipLaunchKernelGGL((attention_kernel<false, true>), grid, dim3(256), 0, ctx->stream, a, plan);
  else
    hipLaunchKernelGGL((attention_kernel<false, false>), grid, dim3(256), 0, ctx->stream, a, plan);
  FOCR_HIP_CHECK(hipGetLastError());
  if (slots > 0) {
    split::Args m;
    m.sinks = a.sinks;
    m.out = a.out;
    m.part = a.part;
    m.query_len = a.query_len;
    m.n_heads = a.n_heads;
    m.tiles = tiles;
    m.slots = slots;
    m.merge_end = a.query_len;
    hipLaunchKernelGGL(split::merge_kernel, dim3(static_cast<unsigned>(tiles), static_cast<unsigned>(a.n_heads), split::kMergeSplit),
                       dim3(256), 0, ctx->stream, m, plan);
    FOCR_HIP_CHECK(hipGetLastError());
  }
  return FOCR_OK;
}

}  // namespace

int launch_attention(Ctx *ctx, const float *q, const float *prefix_k, const float *generated_k, const float *v,
                     size_t query_len, size_t prefix_len, size_t total_len, size_t n_heads, size_t n_kv_heads,
                     size_t query_offset, size_t image_start, size_t image_end, const float *sinks, int softmax,
                     int exp_mode, float *out) {
  FOCR_REQUIRE(total_len < (size_t(1) << 30) && n_heads < 65536, FOCR_E_SHAPE, "attention shape too large");
  AttnArgs a;
  a.prefix_k = prefix_k;
  a.generated_k = generated_k;
  a.v = v;
  a.sinks = sinks;
  a.prefix_len = static_cast<int>(prefix_len);
  a.total_len = static_cast<int>(total_len);
  a.n_heads = static_cast<int>(n_heads);
  a.n_kv_heads = static_cast<int>(n_kv_heads);
  a.image_start = static_cast<int>(image_start);
  a.image_end = static_cast<int>(image_end);
  // Query rows are independent: longer calls run as several launches of at
  // most kMaxTiles query tiles (the plan table's size).
  const size_t per_launch = static_cast<size_t>(kMaxTiles) * kQueries;
  for (size_t q0 = 0; q0 < query_len; q0 += per_launch) {
    const size_t n = query_len - q0 < per_launch ? query_len - q0 : per_launch;
    a.q = q + q0 * n_heads * 64;
    a.out = out + q0 * n_heads * 64;
    a.query_len = static_cast<int>(n);
    a.query_offset = static_cast<int>(query_offset + q0);
    const int rc = launch_tiles(ctx, a, softmax, exp_mode);
    if (rc != FOCR_OK) return rc;
  }
  return FOCR_OK;
}

int launch_attention_split(Ctx *ctx, const float *q, const float *k, const float *v, size_t query_len,
                           size_t n_heads, size_t n_kv_heads, size_t image_start, size_t image_end, const float *sinks,
                           int softmax, int exp_mode, float *out) {
  FOCR_REQUIRE(query_len < (size_t(1) << 30) && n_heads < 65536, FOCR_E_SHAPE, "attention shape too large");
  const size_t ktiles = (query_len + kKeys - 1) / kKeys;
  const size_t kplane = n_heads * ktiles * 256, vplane = n_kv_heads * ktiles * 256;  // uint4 per plane
  // Scratch: K planes, V planes, the K tiles' exponents, the V dims' maxima
  // and the non-finite flag after them.
  const size_t planes_bytes = 2 * (kplane + vplane) * sizeof(uint4);
  const size_t kexp_bytes = (n_heads * ktiles * sizeof(int) + 255) / 256 * 256;
  const size_t vmax_bytes = ((n_kv_heads * 64 + 1) * sizeof(unsigned) + 255) / 256 * 256;
  const size_t kv_bytes = planes_bytes + kexp_bytes + vmax_bytes;
  AttnArgs a;
  a.prefix_k = k;
  a.generated_k = nullptr;
  a.v = v;
  a.sinks = sinks;
  a.prefix_len = static_cast<int>(query_len);
  a.total_len = static_cast<int>(query_len);
  a.n_heads = static_cast<int>(n_heads);
  a.n_kv_heads = static_cast<int>(n_kv_heads);
  a.image_start = static_cast<int>(image_start);
  a.image_end = static_cast<int>(image_end);
  uint4 *kp = nullptr, *vp = nullptr;
  int *kexp = nullptr;
  unsigned *vmax = nullptr, *nonfinite = nullptr;
  auto pair_kv = [&]() -> int {
    char *base = static_cast<char *>(ctx->scratch);
    kp = reinterpret_cast<uint4 *>(base);
    vp = kp + 2 * kplane;
    kexp = reinterpret_cast<int *>(base + planes_bytes);
    vmax = reinterpret_cast<unsigned *>(base + planes_bytes + kexp_bytes);
    const int nv = static_cast<int>(n_kv_heads * 64);
    nonfinite = vmax + nv;
    hipLaunchKernelGGL(pair_zero_kernel, dim3(static_cast<unsigned>((nv + 64) / 64)), dim3(64), 0, ctx->stream, vmax,
                       nv + 1);
    FOCR_HIP_CHECK(hipGetLastError());
    hipLaunchKernelGGL(pair_vmax_kernel, dim3(static_cast<unsigned>(n_kv_heads), static_cast<unsigned>((query_len + 127) / 128)),
                       dim3(256), 0, ctx->stream, v, static_cast<int>(query_len), static_cast<int>(n_kv_heads), vmax,
                       nonfinite);
    FOCR_HIP_CHECK(hipGetLastError());
    hipLaunchKernelGGL(pair_kv_kernel, dim3(static_cast<unsigned>(ktiles), static_cast<unsigned>(n_heads)), dim3(256),
                       0, ctx->stream, k, v, static_cast<int>(query_len), static_cast<int>(n_heads),
                       static_cast<int>(n_kv_heads), static_cast<int>(ktiles), vmax, kp, vp, kexp, nonfinite);
    FOCR_HIP_CHECK(hipGetLastError());
    return FOCR_OK;
  };
  int rc = ensure_scratch(ctx, kv_bytes);
  if (rc != FOCR_OK) return rc;
  rc = pair_kv();
  if (rc != FOCR_OK) return rc;
  // Query rows in launches of at most kMaxTiles query tiles, each with its
  // split plan (parts of whole 32-key tiles) and merge.
  const size_t per_launch = static_cast<size_t>(kMaxTiles) * kQueries;
  for (size_t q0 = 0; q0 < query_len; q0 += per_launch) {
    const int n = static_cast<int>(query_len - q0 < per_launch ? query_len - q0 : per_launch);
    const int tiles = (n + kQueries - 1) / kQueries;
    split::Plan plan;
    int slots = 0;
    const int items = split::make_plan(plan, tiles, n, static_cast<int>(q0), a.image_start, a.image_end, a.n_heads,
                                       kKeys, split::kSplitItemsPair, &slots);
    a.q = q + q0 * n_heads * 64;
    a.out = out + q0 * n_heads * 64;
    a.query_len = n;
    a.query_offset = static_cast<int>(q0);
    a.tiles = tiles;
    a.slots = slots;
    a.part = nullptr;
    if (slots > 0) {
      const size_t part_bytes = static_cast<size_t>(slots) * n_heads * kQueries * 66 * sizeof(float);
      // The planes stay at the front of the scratch; growing it would
      // discard them, so grow first and write them again.
      if (ctx->scratch_bytes < kv_bytes + part_bytes) {
        rc = ensure_scratch(ctx, kv_bytes + part_bytes);
        if (rc != FOCR_OK) return rc;
        rc = pair_kv();
        if (rc != FOCR_OK) return rc;
      }
      a.part = reinterpret_cast<float *>(static_cast<char *>(ctx->scratch) + kv_bytes);
    }
    const dim3 grid(static_cast<unsigned>(items), static_cast<unsigned>(n_heads));
    const int kt = static_cast<int>(ktiles);
    if (softmax == FOCR_SOFTMAX_STATIC) {
      hipLaunchKernelGGL((attention_pair_kernel<true, true>), grid, dim3(256), 0, ctx->stream, a, kp, vp, kexp, vmax,
                         nonfinite, kplane, vplane, kt, plan);
    } else if (exp_mode == FOCR_EXP_FAST) {
      hipLaunchKernelGGL((attention_pair_kernel<false, true>), grid, dim3(256), 0, ctx->stream, a, kp, vp, kexp, vmax,
                         nonfinite, kplane, vplane, kt, plan);
    } else {
      hipLaunchKernelGGL((attention_pair_kernel<false, false>), grid, dim3(256), 0, ctx->stream, a, kp, vp, kexp, vmax,
                         nonfinite, kplane, vplane, kt, plan);
    }
    FOCR_HIP_CHECK(hipGetLastError());
    if (slots > 0) {
      split::Args m;
      m.sinks = a.sinks;
      m.out = a.out;
      m.part = a.part;
      m.query_len = a.query_len;
      m.n_heads = a.n_heads;
      m.tiles = tiles;
      m.slots = slots;
      m.merge_end = a.query_len;
      hipLaunchKernelGGL(split::merge_kernel,
                         dim3(static_cast<unsigned>(tiles), static_cast<unsigned>(a.n_heads), split::kMergeSplit),
                         dim3(256), 0, ctx->stream, m, plan);
      FOCR_HIP_CHECK(hipGetLastError());
    }
  }
  return FOCR_OK;
}

}  // namespace focr
