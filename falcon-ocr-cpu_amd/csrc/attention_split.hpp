// Key-range splitting of the prefill attention kernels (FP32 and BF16).
//
// A 128-query tile of a causal or image-prefixed prefill sees between 128 and
// the whole context's keys, so one workgroup per tile leaves the chip idle
// while the last (longest) tiles finish. Each tile's visible keys are split
// into equal work items (about `target_items` items per call, at least
// kMinChunkKeys keys each); an item runs the tile's online softmax over its keys only and,
// when its tile is split, stores the unnormalized state (max, denominator,
// output) per query row. merge_kernel combines the parts of a row in part
// order — M = max of the maxima, den = sum den_p exp(m_p - M),
// o = sum o_p exp(m_p - M) — and applies the final step of
// prefill64.rs:468-479: lse = M + ln(den), out = (o / den) / (1 + exp(sink - lse)).
// A static-softmax part has no shift and stores max 0 (weights exp(0) = 1).
#pragma once

#include "focr_internal.hpp"

namespace focr {
namespace split {

constexpr int kQueries = 128;   // query rows per tile
constexpr int kMaxTiles = 256;  // plan table size: 32,768 query rows per launch
// Target work items per call. The FP32 kernel's items are long (about 3 per
// workgroup slot balance the tail); the BF16 kernel's are about five times
// shorter, so fewer, larger parts (less partial-state traffic and merge
// work) measure faster there. The FP16-pair kernel's items are about half
// as long as the FP32 kernel's; 2,048 to 4,096 items measured within noise
// of each other at 6,544 and 16,320 rows (1,536: 5-15 % slower).
constexpr long long kSplitItemsF32 = 3072;
constexpr long long kSplitItemsBf16 = 1536;
constexpr long long kSplitItemsPair = 3072;
constexpr long long kMinChunkKeys = 1024;

// Work plan (computed on the host, passed by value): query tiles in dispatch
// order i (tile tiles - 1 - i: the latest, longest tiles first), each split
// into parts of equal size.
struct Plan {
  int first[kMaxTiles + 1];  // first work item of the i-th tile; first[tiles] = items
  int slot[kMaxTiles];       // first partial slot of the i-th tile if it is split
  int keys[kMaxTiles];       // keys per part of the i-th tile
};

struct Args {
  const float *sinks;
  float *out;
  float *part;  // [slot][head][128 rows][64] outputs, then [slot][head][128][2] (max, den)
  int query_len, n_heads, tiles, slots;
  int merge_end;  // rows at or past it are written by another kernel
};

// Keys [0, end) that query tile `tile` sees (tile_span, prefill64/span.rs:9-20).
__host__ __device__ inline int tile_visible_end(int tile, int query_len, int query_offset, int image_start,
                                                int image_end) {
  const int first_query = tile * kQueries;
  const int queries = query_len - first_query < kQueries ? query_len - first_query : kQueries;
  const int first_abs = query_offset + first_query, last_abs = first_abs + queries - 1;
  const bool intersects = first_abs < image_end && last_abs >= image_start;
  return intersects ? (last_abs + 1 > image_end ? last_abs + 1 : image_end) : last_abs + 1;
}

// Builds the plan for `tiles` (<= kMaxTiles) tiles; part sizes are multiples
// of `align` keys. Returns the number of work items; *slots = partial slots.
inline int make_plan(Plan &plan, int tiles, int query_len, int query_offset, int image_start, int image_end,
                     int n_heads, int align, long long target_items, int *slots_out) {
  long long total = 0;
  int vis[kMaxTiles], most = 0;
  for (int t = 0; t < tiles; t++) {
    vis[t] = tile_visible_end(t, query_len, query_offset, image_start, image_end);
    total += vis[t];
    most = vis[t] > most ? vis[t] : most;
  }
  const long long want = total * static_cast<long long>(n_heads) / target_items;
  long long chunk = ((want > kMinChunkKeys ? want : kMinChunkKeys) + align - 1) / align * align;
  // Tiles of nearly equal cost (an all-image or short prefill) balance by
  // themselves: splitting them would only add the merge traffic.
  if (5LL * most <= 6LL * total / (tiles > 0 ? tiles : 1)) chunk = most;
  int items = 0, slots = 0;
  for (int i = 0; i < tiles; i++) {
    const int end = vis[tiles - 1 - i];
    const int want_parts = static_cast<int>((end + chunk - 1) / chunk);
    const int per = ((end + want_parts - 1) / want_parts + align - 1) / align * align;
    const int parts = (end + per - 1) / per;  // every part starts before `end`
    plan.first[i] = items;
    plan.slot[i] = parts > 1 ? slots : -1;
    plan.keys[i] = per;
    items += parts;
    slots += parts > 1 ? parts : 0;
  }
  plan.first[tiles] = items;
  *slots_out = slots;
  return items;
}

// This workgroup's work item: plan order and part.
struct Item {
  int order, part, parts, key_begin, keys;
};
__device__ inline Item find_item(const Plan &plan, int tiles, int item) {
  int lo = 0, hi = tiles - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (plan.first[mid] <= item) lo = mid; else hi = mid - 1;
  }
  Item it;
  it.order = lo;
  it.part = item - plan.first[lo];
  it.parts = plan.first[lo + 1] - plan.first[lo];
  it.keys = plan.keys[lo];
  it.key_begin = it.part * it.keys;
  return it;
}

// Where part `it` of head `head` stores row `row_in_tile`'s state.
__device__ inline float *part_out(const Args &a, const Plan &plan, const Item &it, int head, int row_in_tile) {
  const size_t slot = static_cast<size_t>(plan.slot[it.order] + it.part) * a.n_heads + head;
  return a.part + (slot * kQueries + row_in_tile) * 64;
}
__device__ inline float2 *part_md(const Args &a, const Plan &plan, const Item &it, int head, int row_in_tile) {
  const size_t slot = static_cast<size_t>(plan.slot[it.order] + it.part) * a.n_heads + head;
  return reinterpret_cast<float2 *>(a.part + static_cast<size_t>(a.slots) * a.n_heads * kQueries * 64) +
         slot * kQueries + row_in_tile;
}

// Grid (tiles, heads, kMergeSplit): a workgroup merges kQueries /
// kMergeSplit rows of one tile and head (unsplit tiles exit), eight threads
// per row, each 8 of the 64 dims. The parts' maxima are read first, then
// their outputs kMergeBatch parts at a time (all loads of a batch in flight
// together), added in part order.
constexpr int kMergeSplit = 4;
constexpr int kMergeBatch = 4;
static __global__ __launch_bounds__(256) void merge_kernel(Args a, Plan plan) {
  const int order = blockIdx.x, head = blockIdx.y;
  const int parts = plan.first[order + 1] - plan.first[order];
  if (parts <= 1) return;
  const int row_in_tile = blockIdx.z * (kQueries / kMergeSplit) + (threadIdx.x >> 3), slice = threadIdx.x & 7;
  const int row = (a.tiles - 1 - order) * kQueries + row_in_tile;
  if (row >= a.merge_end) return;
  const float2 *md = reinterpret_cast<const float2 *>(a.part + static_cast<size_t>(a.slots) * a.n_heads * kQueries * 64);
  const size_t slot0 = static_cast<size_t>(plan.slot[order]) * a.n_heads + head;
  const size_t pstride = static_cast<size_t>(a.n_heads);  // slots between consecutive parts of a tile and head
  const float ninf = -__builtin_inff();
  float big = ninf;
  for (int p0 = 0; p0 < parts; p0 += kMergeBatch) {
    float2 m[kMergeBatch];
#pragma unroll
    for (int j = 0; j < kMergeBatch; j++) {
      const int p = p0 + j < parts ? p0 + j : parts - 1;
      m[j] = md[(slot0 + p * pstride) * kQueries + row_in_tile];
    }
#pragma unroll
    for (int j = 0; j < kMergeBatch; j++)
      if (p0 + j < parts) big = __builtin_fmaxf(big, m[j].x);
  }
  float den = 0.0f;
  float4 o[2] = {make_float4(0.f, 0.f, 0.f, 0.f), make_float4(0.f, 0.f, 0.f, 0.f)};
  for (int p0 = 0; p0 < parts; p0 += kMergeBatch) {
    float2 m[kMergeBatch];
    float4 v[kMergeBatch][2];
#pragma unroll
    for (int j = 0; j < kMergeBatch; j++) {
      const int p = p0 + j < parts ? p0 + j : parts - 1;
      const size_t slot = slot0 + p * pstride;
      m[j] = md[slot * kQueries + row_in_tile];
      const float4 *src = reinterpret_cast<const float4 *>(a.part + (slot * kQueries + row_in_tile) * 64 + 8 * slice);
      v[j][0] = src[0];
      v[j][1] = src[1];
    }
#pragma unroll
    for (int j = 0; j < kMergeBatch; j++) {
      if (p0 + j >= parts) break;
      const float f = m[j].x == ninf ? 0.0f : expf_acc(m[j].x - big);
      den = den + m[j].y * f;
#pragma unroll
      for (int i = 0; i < 2; i++)
        o[i] = make_float4(fmaf_(v[j][i].x, f, o[i].x), fmaf_(v[j][i].y, f, o[i].y), fmaf_(v[j][i].z, f, o[i].z),
                           fmaf_(v[j][i].w, f, o[i].w));
    }
  }
  const float lse = big + logf_acc(den);
  const float sink_scale = __fdiv_rn(1.0f, 1.0f + expf_acc(a.sinks[head] - lse));
  float4 *dst = reinterpret_cast<float4 *>(a.out + (static_cast<size_t>(row) * a.n_heads + head) * 64 + 8 * slice);
#pragma unroll
  for (int i = 0; i < 2; i++)
    dst[i] = make_float4(__fmul_rn(__fdiv_rn(o[i].x, den), sink_scale), __fmul_rn(__fdiv_rn(o[i].y, den), sink_scale),
                         __fmul_rn(__fdiv_rn(o[i].z, den), sink_scale), __fmul_rn(__fdiv_rn(o[i].w, den), sink_scale));
}

}  // namespace split
}  // namespace focr
