// The sealed split KV cache (Kv::Q8 / Kv::Q16, src/quant/kv.rs) and decode
// attention over it.
//
// Sealing turns the compact FP32 prefix cache into group-major records, one
// per (KV group g, position t): [T 0..32 | S(2g) 32..64 | S(2g+1) 64..96 |
// V 96..160], the temporal key half shared by the two query heads of the
// pair, each head's spatial half and the value (kv.rs:1-24). Every 32-element
// block is coded against the smallest BF16 step at or above absmax / 127
// (Q8) or absmax / 32767 (Q16), codes rounded to nearest even in f64 and
// clamped (codec.rs:9-86). Generated positions go to 128-element tail
// records [K | V] per group in the same format (push_unique, kv.rs:451-515).
// Decoded values are code * step, exactly as the reference's Records::value.
//
// Device layout: record = the codes, then the BF16 steps (5 per prefix
// record, 4 per tail record), padded to a multiple of 16 bytes (Q8: 176 and
// 144 bytes; Q16: 336 and 272). Prefix records [group][position], tail
// records [group][capacity].
//
// Seal and append code one element per lane (a 32-element block is one
// half-wave; its absmax is a lane exchange), so a decode step's append is a
// single short kernel.
//
// Decode: one workgroup task per (group, key chunk) serves both heads of the
// pair (the record is read once for both); its four waves take interleaved
// 16-key iterations with the compact decode kernel's lane map (lane group
// lg = lane / 16 takes keys 4i + lg, lane lp = lane % 16 dims 4lp..4lp+3),
// every lane reading its codes at offsets selected without branches. Online
// softmax per (head, row), the four waves merged in a fixed order through
// LDS, then the shared combine kernel. With the cache's fast exp
// (SplitPrefix::with_fast_exp, kv.rs:423; the polynomial exp of the
// reference's exp_shifted, decode.rs:346-347) the per-key probabilities
// p = exp(s - max) use the hardware exp2 of log2(e) * x instead of the device
// libm expf, within a few ulp of the reference's exp_poly; the block rescale
// and the chunk merge keep expf, as the reference keeps the platform exp
// there. Roofline: HBM; bytes per call = the visible
// records (Q8: 176 bytes per group and prefix position, 8 groups = 1,408
// bytes per position against 6,144 for the FP32 compact cache).
#include <mutex>
#include <vector>

#include "decode_common.hpp"

// Partial softmax states of focr_kv_attention_decode_noalloc: a fixed
// device-resident array instead of the context scratch, so that the call
// allocates nothing. Every GPU the library runs on holds its own copy for
// the life of the process. In host code `scratch` names a host-side stand-in,
// never device memory: kernels get the per-device address that
// hipGetSymbolAddress returns (noalloc_scratch below).
constexpr size_t kNoAllocScratchBytes = size_t(4608) << 10;  // 4.5 MiB
static __device__ __align__(256) float scratch[kNoAllocScratchBytes / sizeof(float)];

namespace focr {

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
float *g_scratch_ptr[kMaxDevices] = {};
}  // namespace

// Resolves this device's address of `scratch`, once per device, with the
// device current (called by focr_ctx_create).
int noalloc_scratch_init(int device) {
  FOCR_REQUIRE(device >= 0 && device < kMaxDevices, FOCR_E_UNSUPPORTED, "device index beyond the no-alloc table");
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch_ptr[device]) return FOCR_OK;
  int current = -1;
  FOCR_HIP_CHECK(hipGetDevice(&current));
  FOCR_REQUIRE(current == device, FOCR_E_ARG, "noalloc_scratch_init: the device must be current");
  void *ptr = nullptr;
  FOCR_HIP_CHECK(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)));
  FOCR_REQUIRE(ptr, FOCR_E_HIP, "hipGetSymbolAddress returned no address for the no-alloc scratch");
  g_scratch_ptr[device] = static_cast<float *>(ptr);
  return FOCR_OK;
}

namespace {
float *noalloc_scratch(int device) {
  if (device < 0 || device >= kMaxDevices) return nullptr;
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  return g_scratch_ptr[device];
}
}  // namespace

struct KvSplit {
  int bits = 8;
  int n_heads = 0, n_kv = 0;
  size_t prefix_len = 0, capacity = 0, tail_len = 0;
  size_t record_bytes = 0, tail_bytes = 0;
  unsigned char *records = nullptr;  // [n_kv][prefix_len][record_bytes]
  unsigned char *tail = nullptr;     // [n_kv][capacity - prefix_len][tail_bytes]
  uint32_t *error = nullptr;         // seal's refusal flags
  size_t device_bytes = 0;
  bool fast_exp = false;  // SplitPrefix::fast_exp (kv.rs:168-170)
};

namespace {

using namespace decode;

constexpr int kRecord = 160, kTail = 128;

__device__ __forceinline__ float bf16_widen(uint16_t bits) { return __uint_as_float(static_cast<uint32_t>(bits) << 16); }

// The smallest BF16 at or above a finite scale >= 0, or the NaN pattern.
__device__ __forceinline__ uint16_t bf16_up(float scale) {
  if (scale != scale) return 0x7FC0;
  const uint32_t bits = __float_as_uint(scale);
  const uint16_t high = static_cast<uint16_t>(bits >> 16);
  return (bits & 0xFFFFu) ? static_cast<uint16_t>(high + 1) : high;
}

// round_clamped(value / step): clamp to +-limit in f64, round to nearest
// even; NaN gives 0 (Rust's saturating cast); a zero step gives 0.
__device__ __forceinline__ int code_of(float value, float step, double limit) {
  if (step == 0.0f) return 0;
  double x = static_cast<double>(value) / static_cast<double>(step);
  if (x != x) return 0;
  x = x < -limit ? -limit : (x > limit ? limit : x);
  return static_cast<int>(rint(x));
}

// Codes one 32-element block held by the 32 lanes of a half-wave (lane & 31
// = element; every lane of the wave takes part in the exchanges). The step
// (q8_scale / q16_scale) is absmax / limit in f64 rounded to f32, at least
// the smallest subnormal, 0 for an all-zero block, stored as the smallest
// BF16 at or above it; `nan_step` stores the NaN pattern instead. The max is
// exact, so the exchange order does not matter. Returns the code; `step`
// receives the stored BF16. DPP: the exchanges by v_permlane16_swap (the
// half's two rows) and DPP within the rows instead of five LDS permutes.
template <bool DPP = false>
__device__ __forceinline__ int code_lane(float x, bool nan_step, double limit, uint16_t &stored) {
  float mx = __builtin_fmaxf(0.0f, fabsf(x));  // a NaN element counts as 0
  if constexpr (DPP) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(mx), __float_as_uint(mx), false, false);
    mx = __builtin_fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));  // lanes i and i ^ 16
    mx = __builtin_fmaxf(mx, dpp<0xB1>(mx));   // quad_perm [1,0,3,2]
    mx = __builtin_fmaxf(mx, dpp<0x4E>(mx));   // quad_perm [2,3,0,1]
    mx = __builtin_fmaxf(mx, dpp<0x141>(mx));  // row_half_mirror
    mx = __builtin_fmaxf(mx, dpp<0x140>(mx));  // row_mirror
  } else {
#pragma unroll
    for (int mask = 1; mask < 32; mask *= 2) mx = __builtin_fmaxf(mx, xor_lane(mx, mask));
  }
  float step = 0.0f;
  if (mx != 0.0f) {
    step = static_cast<float>(static_cast<double>(mx) / limit);
    step = step > 1.40129846e-45f ? step : 1.40129846e-45f;
  }
  stored = bf16_up(nan_step ? __builtin_nanf("") : step);
  return code_of(x, bf16_widen(stored), limit);
}

// Whether any lane of this lane's half-wave has `pred` set.
__device__ __forceinline__ bool half_any(bool pred) {
  const unsigned long long b = __ballot(pred);
  return ((b >> (threadIdx.x & 32)) & 0xffffffffull) != 0;
}

enum : uint32_t { kErrPair = 1, kErrNonFinite = 2, kErrOverflow = 4 };

struct SealArgs {
  const float *k, *v;
  unsigned char *records;
  uint32_t *error;
  int prefix_len, n_heads, n_kv, record_bytes;
};

// Records per seal_kernel lane.
constexpr int kSealPer = 8;

// Lane = element e of kSealPer records, `pass` records apart (group-major
// records of 160 = 5 blocks of 32, so every block is one aligned half-wave):
// gathers the elements (every load issued before any element is coded, so
// a wave has kSealPer loads in flight instead of one), checks the pair
// sharing (block 0) and finiteness, codes them.
template <typename C>
__global__ __launch_bounds__(256) void seal_kernel(SealArgs a, long pass) {
  const long idx = static_cast<long>(blockIdx.x) * 256 + threadIdx.x;
  const long nrec = static_cast<long>(a.n_kv) * a.prefix_len;
  const long rec0 = idx / kRecord;
  const int e = static_cast<int>(idx % kRecord);
  float x[kSealPer], pair[kSealPer];
  bool valid[kSealPer];
#pragma unroll
  for (int j = 0; j < kSealPer; j++) {
    const long record = rec0 + j * pass;
    valid[j] = rec0 < pass && record < nrec;
    const long r = valid[j] ? record : 0;
    const int g = static_cast<int>(r / a.prefix_len), t = static_cast<int>(r % a.prefix_len);
    const float *ka = a.k + (static_cast<size_t>(t) * a.n_heads + 2 * g) * 64;
    const float *src =
        e < 64 ? ka + e : e < 96 ? ka + 32 + e : a.v + (static_cast<size_t>(t) * a.n_kv + g) * 64 + e - 96;
    x[j] = valid[j] ? *src : 0.0f;
    pair[j] = valid[j] && e < 32 ? ka[64 + e] : 0.0f;
  }
  uint32_t err = 0;
  const double limit = sizeof(C) == 1 ? 127.0 : 32767.0;
#pragma unroll
  for (int j = 0; j < kSealPer; j++) {
    if (valid[j] && !__builtin_isfinite(x[j])) err |= kErrNonFinite;
    if (valid[j] && e < 32 && __float_as_uint(x[j]) != __float_as_uint(pair[j])) err |= kErrPair;
    uint16_t stored;
    const int code = code_lane<true>(x[j], false, limit, stored);
    if (valid[j]) {
      unsigned char *rec = a.records + static_cast<size_t>(rec0 + j * pass) * a.record_bytes;
      reinterpret_cast<C *>(rec)[e] = static_cast<C>(code);
      if ((e & 31) == 0) reinterpret_cast<uint16_t *>(rec + kRecord * sizeof(C))[e >> 5] = stored;
      if (!__builtin_isfinite(static_cast<float>(code) * bf16_widen(stored))) err |= kErrOverflow;
    }
  }
  if (err) atomicOr(a.error, err);
}

struct AppendArgs {
  const float *k, *v;  // [rows][n_kv][64]
  unsigned char *tail;
  int n_kv, tail_capacity, first, rows, tail_bytes;
};

// One lane per tail-record element (128 = 4 blocks, so the grid is whole
// waves): a block holding a non-finite value is coded against the NaN step.
template <typename C>
__global__ __launch_bounds__(256) void append_kernel(AppendArgs a) {
  const int idx = blockIdx.x * 256 + threadIdx.x;
  const bool valid = idx < a.rows * a.n_kv * kTail;
  const int e = idx % kTail, g = (idx / kTail) % a.n_kv, r = idx / (kTail * a.n_kv);
  const float *src = (e < 64 ? a.k + e : a.v + e - 64) + (static_cast<size_t>(r) * a.n_kv + g) * 64;
  const float x = valid ? *src : 0.0f;
  const bool nonfinite = half_any(!__builtin_isfinite(x));
  uint16_t stored;
  const int code = code_lane(x, nonfinite, sizeof(C) == 1 ? 127.0 : 32767.0, stored);
  if (valid) {
    unsigned char *rec = a.tail + (static_cast<size_t>(g) * a.tail_capacity + a.first + r) * a.tail_bytes;
    reinterpret_cast<C *>(rec)[e] = static_cast<C>(code);
    if ((e & 31) == 0) reinterpret_cast<uint16_t *>(rec + kTail * sizeof(C))[e >> 5] = stored;
  }
}

struct RowAppendArgs {
  const float *qkv, *rope;  // [rows][qdim + 2 kdim], [rows][n_heads][32] (cos, sin)
  float *q;                 // [rows][n_heads][64]
  unsigned char *tail;
  int n_heads, n_kv, tail_capacity, first, tail_bytes;
};

// The decode row step over a sealed cache, one workgroup of 16 waves per
// row: the query heads normalized and rotated as split_norm_rope does (to q),
// the unique key heads likewise (head g * repeat's factors,
// append_unique_heads) and the values copied, both coded straight into the
// row's tail records (push_unique) instead of through an FP32 buffer. Every
// value is the unfused path's bit for bit (the same norm_rope, the same
// code_lane). Jobs of one wave each, lane = element: n_heads queries, n_kv
// keys (two blocks each), n_kv value halves of records; a wave loads its
// (at most two) jobs before computing.
constexpr int kRowWaves = 16;

template <typename C>
__global__ __launch_bounds__(1024) void row_append_kernel(RowAppendArgs a) {
  const int row = blockIdx.x;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int qdim = a.n_heads * 64, kdim = a.n_kv * 64, repeat = a.n_heads / a.n_kv;
  const float *src = a.qkv + static_cast<size_t>(row) * (qdim + 2 * kdim);
  const float2 *rope = reinterpret_cast<const float2 *>(a.rope) + static_cast<size_t>(row) * a.n_heads * 32;
  const double limit = sizeof(C) == 1 ? 127.0 : 32767.0;
  const int jobs = a.n_heads + 2 * a.n_kv;
  // Job j: query head j, key head j - n_heads, or the values of group
  // j - n_heads - n_kv.
  auto load = [&](int job, float &x, float2 &f) {
    if (job < a.n_heads) {
      x = src[job * 64 + lane];
      f = rope[job * 32 + lane / 2];
    } else if (job < a.n_heads + a.n_kv) {
      const int g = job - a.n_heads;
      x = src[qdim + g * 64 + lane];
      f = rope[g * repeat * 32 + lane / 2];
    } else {
      x = src[qdim + kdim + (job - a.n_heads - a.n_kv) * 64 + lane];
    }
  };
  auto finish = [&](int job, float x, float2 f) {
    if (job < a.n_heads) {
      a.q[static_cast<size_t>(row) * qdim + job * 64 + lane] = norm_rope(x, f, lane);
      return;
    }
    const bool key = job < a.n_heads + a.n_kv;
    const int g = key ? job - a.n_heads : job - a.n_heads - a.n_kv;
    const float y = key ? norm_rope(x, f, lane) : x;
    uint16_t stored;
    const int code = code_lane(y, half_any(!__builtin_isfinite(y)), limit, stored);
    unsigned char *rec = a.tail + (static_cast<size_t>(g) * a.tail_capacity + a.first + row) * a.tail_bytes;
    const int e = (key ? 0 : 64) + lane;
    reinterpret_cast<C *>(rec)[e] = static_cast<C>(code);
    if ((e & 31) == 0) reinterpret_cast<uint16_t *>(rec + kTail * sizeof(C))[e >> 5] = stored;
  };
  constexpr int kHoist = 2;
  float xs[kHoist];
  float2 fs[kHoist];
#pragma unroll
  for (int i = 0; i < kHoist; i++) {
    const int job = wave + kRowWaves * i;
    fs[i] = make_float2(0.0f, 0.0f);
    if (job < jobs) load(job, xs[i], fs[i]);
  }
#pragma unroll
  for (int i = 0; i < kHoist; i++) {
    const int job = wave + kRowWaves * i;
    if (job < jobs) finish(job, xs[i], fs[i]);
  }
  for (int job = wave + kRowWaves * kHoist; job < jobs; job += kRowWaves) {
    float x;
    float2 f = make_float2(0.0f, 0.0f);
    load(job, x, f);
    finish(job, x, f);
  }
}

struct DequantArgs {
  const unsigned char *records, *tail;
  float *prefix_k, *values, *generated_k;
  int prefix_len, tail_len, tail_capacity, n_heads, n_kv, record_bytes, tail_bytes;
};

// The decoded cache in the compact layout (kv.rs dequantized_compact plus
// the tail): one thread per (position, group, element).
template <typename C>
__global__ __launch_bounds__(256) void dequantize_kernel(DequantArgs a) {
  const long idx = static_cast<long>(blockIdx.x) * 256 + threadIdx.x;
  const long prefix_items = static_cast<long>(a.prefix_len) * a.n_kv * kRecord;
  const long tail_items = static_cast<long>(a.tail_len) * a.n_kv * kTail;
  if (idx < prefix_items) {
    const int e = static_cast<int>(idx % kRecord);
    const long rg = idx / kRecord;
    const int g = static_cast<int>(rg % a.n_kv), t = static_cast<int>(rg / a.n_kv);
    const unsigned char *rec = a.records + (static_cast<size_t>(g) * a.prefix_len + t) * a.record_bytes;
    const float x = static_cast<float>(reinterpret_cast<const C *>(rec)[e]) *
                    bf16_widen(reinterpret_cast<const uint16_t *>(rec + kRecord * sizeof(C))[e / 32]);
    float *k0 = a.prefix_k + (static_cast<size_t>(t) * a.n_heads + 2 * g) * 64;
    if (e < 32) {
      k0[e] = x;
      k0[64 + e] = x;
    } else if (e < 64) {
      k0[e] = x;
    } else if (e < 96) {
      k0[64 + e - 32] = x;
    } else {
      a.values[(static_cast<size_t>(t) * a.n_kv + g) * 64 + e - 96] = x;
    }
  } else if (idx < prefix_items + tail_items) {
    const long j = idx - prefix_items;
    const int e = static_cast<int>(j % kTail);
    const long rg = j / kTail;
    const int g = static_cast<int>(rg % a.n_kv), i = static_cast<int>(rg / a.n_kv);
    const unsigned char *rec = a.tail + (static_cast<size_t>(g) * a.tail_capacity + i) * a.tail_bytes;
    const float x = static_cast<float>(reinterpret_cast<const C *>(rec)[e]) *
                    bf16_widen(reinterpret_cast<const uint16_t *>(rec + kTail * sizeof(C))[e / 32]);
    if (e < 64)
      a.generated_k[(static_cast<size_t>(i) * a.n_kv + g) * 64 + e] = x;
    else
      a.values[(static_cast<size_t>(a.prefix_len + i) * a.n_kv + g) * 64 + e - 64] = x;
  }
}

struct SplitDecArgs {
  const unsigned char *records, *tail;
  const float *q;
  float *part_o, *part_md;
  int prefix_len, tail_capacity, n_heads, n_kv, record_bytes, tail_bytes;
  int last;  // positions in the cache; row r sees keys [0, last - rows + r + 1)
  int chunks, tasks;
  // The fused row step (split_scan_kernel with ROW): the row's raw q|k|v, its
  // RoPE factors, where its queries go (optional), and the record to write.
  const float *qkv, *rope;
  float *q_out;
  unsigned char *tail_w;
};

// Four consecutive codes of a record as floats (one 4- or 8-byte load).
template <typename C>
__device__ __forceinline__ float4 codes4(const unsigned char *p) {
  if constexpr (sizeof(C) == 1) {
    const uint32_t w = *reinterpret_cast<const uint32_t *>(p);
    return make_float4(static_cast<float>(static_cast<int8_t>(w & 0xff)), static_cast<float>(static_cast<int8_t>((w >> 8) & 0xff)),
                       static_cast<float>(static_cast<int8_t>((w >> 16) & 0xff)), static_cast<float>(static_cast<int8_t>(w >> 24)));
  } else {
    const uint2 w = *reinterpret_cast<const uint2 *>(p);
    return make_float4(static_cast<float>(static_cast<int16_t>(w.x & 0xffff)), static_cast<float>(static_cast<int16_t>(w.x >> 16)),
                       static_cast<float>(static_cast<int16_t>(w.y & 0xffff)), static_cast<float>(static_cast<int16_t>(w.y >> 16)));
  }
}

__device__ __forceinline__ float4 scale4(float4 c, float s) { return make_float4(c.x * s, c.y * s, c.z * s, c.w * s); }

// A key's (both heads') and value's decoded values for lane lp (dims
// 4lp..4lp+3 of each 64-wide head). Branch-free over the record kind: in a
// prefix record head 2g's key is codes [0, 64) (T then S(2g)) and head
// 2g+1's is T then S(2g+1) = codes [64, 96); a tail record holds one key
// [0, 64) for both heads. The BF16 steps follow the codes, 16-byte aligned.
struct KeyVal {
  float4 k0, k1, v;
};

__device__ __forceinline__ float step_of(uint4 w, int i) {
  const uint32_t word = i < 2 ? w.x : i < 4 ? w.y : i < 6 ? w.z : w.w;
  return bf16_widen(static_cast<uint16_t>((i & 1) ? word >> 16 : word & 0xffffu));
}

template <typename C>
__device__ __forceinline__ KeyVal load_key(const SplitDecArgs &a, int g, int j, int lp) {
  const bool prefix = j < a.prefix_len;
  const unsigned char *rec =
      prefix ? a.records + (static_cast<size_t>(g) * a.prefix_len + j) * a.record_bytes
             : a.tail + (static_cast<size_t>(g) * a.tail_capacity + (j - a.prefix_len)) * a.tail_bytes;
  const int hi = lp >> 3;
  const int k1_at = prefix ? 4 * lp + 32 * hi : 4 * lp;
  const int v_at = (prefix ? 96 : 64) + 4 * lp;
  const uint4 steps = *reinterpret_cast<const uint4 *>(rec + (prefix ? kRecord : kTail) * sizeof(C));
  const float4 c0 = codes4<C>(rec + 4 * lp * sizeof(C));
  const float4 c1 = codes4<C>(rec + k1_at * sizeof(C));
  const float4 cv = codes4<C>(rec + v_at * sizeof(C));
  KeyVal kv;
  kv.k0 = scale4(c0, step_of(steps, hi));
  kv.k1 = scale4(c1, step_of(steps, prefix ? 2 * hi : hi));
  kv.v = scale4(cv, step_of(steps, (prefix ? 3 : 2) + hi));
  return kv;
}

// load_key of a prefix record that sits in LDS at `rec`.
template <typename C>
__device__ __forceinline__ KeyVal lds_key(const unsigned char *rec, int lp) {
  const int hi = lp >> 3;
  const uint4 steps = *reinterpret_cast<const uint4 *>(rec + kRecord * sizeof(C));
  const float4 c0 = codes4<C>(rec + 4 * lp * sizeof(C));
  const float4 c1 = codes4<C>(rec + (4 * lp + 32 * hi) * sizeof(C));
  const float4 cv = codes4<C>(rec + (96 + 4 * lp) * sizeof(C));
  KeyVal kv;
  kv.k0 = scale4(c0, step_of(steps, hi));
  kv.k1 = scale4(c1, step_of(steps, 2 * hi));
  kv.v = scale4(cv, step_of(steps, 3 + hi));
  return kv;
}

constexpr int kKpl = 4;  // keys per lane group per iteration (16 per wave)
constexpr int kRoundKeys = 16 * kWaves;  // positions per workgroup round

typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(1))) const void global_void;

// M: query rows. One workgroup per task (group g, key chunk c) serves heads
// 2g and 2g + 1 in rounds of 64 positions: wave w takes positions 16w ..
// 16w + 15 of each round, and the four waves' states are merged in a fixed
// order through LDS. The round's prefix records (contiguous in HBM) are
// copied to LDS by the LDS-DMA path, 16 bytes per lane, the next round's
// while the current one is scored; generated keys (the tail) and the padding
// keys past the last visible one are read from HBM as before.
template <typename C>
struct RoundBuf {
  static constexpr int kCopies = (kRoundKeys * (kRecord * static_cast<int>(sizeof(C)) + 16) + 4095) / 4096;
  uint4 chunk[256 * kCopies];  // [kCopies][256 threads] x 16 B
};

constexpr float kLog2e = 1.44269504088896340736f;

// p = exp(x) for x <= 0: the exact device expf, or with FAST the hardware
// exp2 (v_exp_f32, 1 ulp) of log2(e) * x.
template <bool FAST>
__device__ __forceinline__ float prob_exp(float x) {
  if constexpr (FAST)
    return __builtin_amdgcn_exp2f(kLog2e * x);
  else
    return expf_acc(x);
}

template <typename C, int M, bool FAST>
__global__ __launch_bounds__(256) void split_partial_kernel(SplitDecArgs a, int iters, int rows) {
  __shared__ float4 s_o[kWaves][2][M][16];
  __shared__ float2 s_md[kWaves][2][M];
  // Two distinct LDS objects, so the compiler sees that reading one does not
  // wait for the copies into the other.
  __shared__ RoundBuf<C> rb0, rb1;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int lg = lane >> 4, lp = lane & 15;
  const int task = blockIdx.x;
  const int c = task % a.chunks, g = task / a.chunks;
  const int key0 = c * iters * 4 * kKpl;
  int vis[M], limit = 0;
#pragma unroll
  for (int r = 0; r < M; r++) {
    vis[r] = a.last - rows + r + 1;
    limit = vis[r] > limit ? vis[r] : limit;
  }
  float4 qv[2][M];
#pragma unroll
  for (int e = 0; e < 2; e++)
#pragma unroll
    for (int r = 0; r < M; r++)
      qv[e][r] = ld4(a.q + (static_cast<size_t>(r) * a.n_heads + 2 * g + e) * 64 + 4 * lp);
  const float ninf = -__builtin_inff();
  float m[2][M], den[2][M];
  float4 o[2][M];
#pragma unroll
  for (int e = 0; e < 2; e++)
#pragma unroll
    for (int r = 0; r < M; r++) {
      m[e][r] = ninf;
      den[e][r] = 0.0f;
      o[e][r] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
  // Round t's copies: chunk q = tid + 256 i of the rows [b, b + 64) of group
  // g's prefix records (b = key0 + 64 t); chunks past the prefix (or a round
  // entirely in the tail) copy the group's first chunk instead, into slots
  // that are never read.
  constexpr int kCopies = RoundBuf<C>::kCopies;
  const int rbytes = a.record_bytes;
  const unsigned char *group_base = a.records + static_cast<size_t>(g) * a.prefix_len * rbytes;
  auto issue = [&](RoundBuf<C> &dst, int t) {
    const int b = key0 + kRoundKeys * t;
    const int in_prefix = a.prefix_len - b;
    const int valid = in_prefix <= 0 ? 0 : (in_prefix < kRoundKeys ? in_prefix : kRoundKeys) * rbytes;
    const unsigned char *src = group_base + static_cast<size_t>(in_prefix > 0 ? b : 0) * rbytes;
#pragma unroll
    for (int i = 0; i < kCopies; i++) {
      const int off = (threadIdx.x + 256 * i) * 16;
      __builtin_amdgcn_global_load_lds((global_void *)(src + (off < valid ? off : 0)),
                                       (lds_void *)(&dst.chunk[64 * wave + 256 * i]), 16, 0, 0);
    }
  };
  auto load = [&](KeyVal (&kb)[kKpl], int it) {
#pragma unroll
    for (int i = 0; i < kKpl; i++) {
      const int j = key0 + 16 * it + 4 * i + lg;
      kb[i] = load_key<C>(a, g, j < limit ? j : 0, lp);
    }
  };
  auto consume = [&](const KeyVal (&kb)[kKpl], int it) {
    float s[2][kKpl][M];
#pragma unroll
    for (int i = 0; i < kKpl; i++) {
      const int j = key0 + 16 * it + 4 * i + lg;
#pragma unroll
      for (int e = 0; e < 2; e++) {
        const float4 k = e == 0 ? kb[i].k0 : kb[i].k1;
#pragma unroll
        for (int r = 0; r < M; r++) {
          float d = qv[e][r].x * k.x;
          d = fmaf_(qv[e][r].y, k.y, d);
          d = fmaf_(qv[e][r].z, k.z, d);
          d = fmaf_(qv[e][r].w, k.w, d);
          d = row_sum16(d) * 0.125f;
          s[e][i][r] = j < vis[r] ? d : ninf;
        }
      }
    }
#pragma unroll
    for (int e = 0; e < 2; e++)
#pragma unroll
      for (int r = 0; r < M; r++) {
        float bmax = s[e][0][r];
#pragma unroll
        for (int i = 1; i < kKpl; i++) bmax = s[e][i][r] > bmax ? s[e][i][r] : bmax;
        const float mn = bmax > m[e][r] ? bmax : m[e][r];
        if (mn == ninf) continue;
        const float rs = m[e][r] == ninf ? 0.0f : expf_acc(m[e][r] - mn);
        den[e][r] = den[e][r] * rs;
        o[e][r] = scale4(o[e][r], rs);
        m[e][r] = mn;
#pragma unroll
        for (int i = 0; i < kKpl; i++) {
          const float p = s[e][i][r] == ninf ? 0.0f : prob_exp<FAST>(s[e][i][r] - mn);
          const float4 v = kb[i].v;
          den[e][r] = den[e][r] + p;
          o[e][r] = make_float4(fmaf_(p, v.x, o[e][r].x), fmaf_(p, v.y, o[e][r].y), fmaf_(p, v.z, o[e][r].z),
                                fmaf_(p, v.w, o[e][r].w));
        }
      }
  };
  // iters is a multiple of kWaves: every wave takes iters / kWaves
  // iterations, one per round. Past the last round the copy repeats it into
  // the free buffer (no branch around the copies: a branch join would make
  // the compiler wait for every copy in flight).
  const int rounds = iters / kWaves;
  auto round = [&](const RoundBuf<C> &cur, RoundBuf<C> &next, int t) __attribute__((always_inline)) {
    __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0): this wave's copies of round t
    __syncthreads();                     // everyone's copies; nobody still reads `next`
    issue(next, t + 1 < rounds ? t + 1 : rounds - 1);
    const int it = kWaves * t + wave, b = key0 + kRoundKeys * t;
    KeyVal kb[kKpl];
    // A round wholly inside the visible prefix is scored from LDS; the
    // round that reaches the tail or the last visible key reads HBM. Each
    // branch consumes its own keys: a key loaded from HBM must not reach
    // past the join, where waiting for it would also wait for the copies.
    if (b + kRoundKeys <= a.prefix_len && b + kRoundKeys <= limit) {
#pragma unroll
      for (int i = 0; i < kKpl; i++)
        kb[i] = lds_key<C>(reinterpret_cast<const unsigned char *>(cur.chunk) + (16 * wave + 4 * i + lg) * rbytes, lp);
      consume(kb, it);
    } else {
      load(kb, it);
      consume(kb, it);
    }
  };
  issue(rb0, 0);
  int t = 0;
  for (; t + 2 <= rounds; t += 2) {
    round(rb0, rb1, t);
    round(rb1, rb0, t + 1);
  }
  if (t < rounds) round(rb0, rb1, t);
  __builtin_amdgcn_s_waitcnt(0x0f70);  // the repeated copies land before LDS is reused
#pragma unroll
  for (int e = 0; e < 2; e++)
#pragma unroll
    for (int r = 0; r < M; r++) {
#pragma unroll
      for (int mask = 16; mask <= 32; mask *= 2) {
        const float m2 = xor_lane(m[e][r], mask), d2 = xor_lane(den[e][r], mask);
        const float4 o2 = make_float4(xor_lane(o[e][r].x, mask), xor_lane(o[e][r].y, mask),
                                      xor_lane(o[e][r].z, mask), xor_lane(o[e][r].w, mask));
        merge(m[e][r], den[e][r], o[e][r], m2, d2, o2);
      }
      if (lg == 0) s_o[wave][e][r][lp] = o[e][r];
      if (lane == 0) s_md[wave][e][r] = make_float2(m[e][r], den[e][r]);
    }
  __syncthreads();
  // Wave w's lanes 16e' + lp merge the four waves for (head e, rows r = w,
  // w + 4): lane group lg < 2 is the head.
  if (lg < 2) {
    const int e = lg;
#pragma unroll
    for (int r = 0; r < M; r++) {
      if (r % kWaves != wave) continue;
      float2 md = s_md[0][e][r];
      float4 acc = s_o[0][e][r][lp];
#pragma unroll
      for (int w = 1; w < kWaves; w++) {
        const float2 md2 = s_md[w][e][r];
        merge(md.x, md.y, acc, md2.x, md2.y, s_o[w][e][r][lp]);
      }
      const size_t slot = (static_cast<size_t>(r) * a.n_heads + 2 * g + e) * a.chunks + c;
      *reinterpret_cast<float4 *>(a.part_o + slot * 64 + 4 * lp) = acc;
      if (lp == 0) *reinterpret_cast<float2 *>(a.part_md + slot * 2) = md;
    }
  }
}

// Code I (0..3) of a 32-bit word of four Q8 codes, or (0..1) of two Q16
// codes, as a float (exact). Plain C: the compiler forms the SDWA conversion
// itself and, unlike for inline assembly, knows it needs no wait state
// before the FMA that reads it.
template <typename C, int I>
__device__ __forceinline__ float word_code(uint32_t w) {
  if constexpr (sizeof(C) == 1)
    return static_cast<float>(static_cast<int8_t>(w >> (8 * I)));
  else
    return static_cast<float>(static_cast<int16_t>(w >> (16 * I)));
}

// The scan for one or two query rows, with the work of a 16-key slice laid
// out so that no lane repeats another's: for the scores, lane (key kk, head
// e, half) forms the dot of its 32 dims of head 2g + e with the key's codes
// (T for half 0, S(2g + e) for half 1 of a prefix record; the key's dims
// 0-31 / 32-63 of a tail record), scaled once by the block's step, and the
// two halves are added across lanes; for the values, lane (dim quad dq, key
// quarter ks) accumulates dims 4dq .. 4dq + 3 of both heads over keys
// 4i + ks with the block's step folded into p. The running max is taken per
// 16-key slice (uniform over the slice's lanes), each score lane keeps its
// own denominator part, and the parts are summed at the end. Tolerance-only
// against the reference's operation order, as the split-K scan already is.
//
// ROW (one row): the decode row step runs in the same launch. Waves 0 and 1
// of every task normalize and rotate the query heads 2g and 2g + 1 from the
// raw q|k|v row (norm_rope, as row_append_kernel), and the task holding the
// new position (the last chunk) codes the group's key and values into the
// new tail record (waves 2, 3) before any round reads it; the other tasks
// never read that record. Queries and records are bitwise the
// row_append_kernel's, so the output is bitwise the unfused pair of calls.
template <typename C, int M, bool FAST, bool ROW = false>
__global__ __launch_bounds__(256) void split_scan_kernel(SplitDecArgs a, int iters, int rows) {
  static_assert(!ROW || M == 1, "the fused row step takes one row");
  __shared__ float4 s_o[kWaves][2][M][16];
  __shared__ float2 s_md[kWaves][2][M];
  __shared__ float2 s_p[kWaves][16][M];  // the slice's probabilities (head 2g, head 2g + 1)
  __shared__ float s_q[2][64];
  __shared__ RoundBuf<C> rb0, rb1;
  constexpr int B = sizeof(C);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int kk = lane & 15, e = (lane >> 4) & 1, half = lane >> 5;
  const int dq = lane & 15, ks = lane >> 4;
  const int task = blockIdx.x;
  const int c = task % a.chunks, g = task / a.chunks;
  const int key0 = c * iters * 4 * kKpl;
  int vis[M], limit = 0;
#pragma unroll
  for (int r = 0; r < M; r++) {
    vis[r] = a.last - rows + r + 1;
    limit = vis[r] > limit ? vis[r] : limit;
  }
  constexpr int kCopies = RoundBuf<C>::kCopies;
  const int rbytes = a.record_bytes;
  const unsigned char *group_base = a.records + static_cast<size_t>(g) * a.prefix_len * rbytes;
  auto issue = [&](RoundBuf<C> &dst, int t) {
    const int b = key0 + kRoundKeys * t;
    const int in_prefix = a.prefix_len - b;
    const int valid = in_prefix <= 0 ? 0 : (in_prefix < kRoundKeys ? in_prefix : kRoundKeys) * rbytes;
    const unsigned char *src = group_base + static_cast<size_t>(in_prefix > 0 ? b : 0) * rbytes;
#pragma unroll
    for (int i = 0; i < kCopies; i++) {
      const int off = (threadIdx.x + 256 * i) * 16;
      __builtin_amdgcn_global_load_lds((global_void *)(src + (off < valid ? off : 0)),
                                       (lds_void *)(&dst.chunk[64 * wave + 256 * i]), 16, 0, 0);
    }
  };
  issue(rb0, 0);
  float qv[M][32];
  if constexpr (ROW) {
    // The row step while round 0's copies are in flight.
    const int qdim = a.n_heads * 64, kdim = a.n_kv * 64, repeat = a.n_heads / a.n_kv;
    const float2 *rope = reinterpret_cast<const float2 *>(a.rope);
    if (wave < 2) {
      const int head = 2 * g + wave;
      const float y = norm_rope(a.qkv[head * 64 + lane], rope[head * 32 + lane / 2], lane);
      s_q[wave][lane] = y;
      if (a.q_out && c == 0) a.q_out[head * 64 + lane] = y;
    } else if (c == a.chunks - 1) {
      const bool key = wave == 2;
      const float x = key ? a.qkv[qdim + g * 64 + lane] : a.qkv[qdim + kdim + g * 64 + lane];
      const float y = key ? norm_rope(x, rope[g * repeat * 32 + lane / 2], lane) : x;
      uint16_t stored;
      const int code = code_lane(y, half_any(!__builtin_isfinite(y)), sizeof(C) == 1 ? 127.0 : 32767.0, stored);
      unsigned char *rec = a.tail_w + static_cast<size_t>(g) * a.tail_capacity * a.tail_bytes;
      const int el = (key ? 0 : 64) + lane;
      reinterpret_cast<C *>(rec)[el] = static_cast<C>(code);
      if ((el & 31) == 0) reinterpret_cast<uint16_t *>(rec + kTail * sizeof(C))[el >> 5] = stored;
    }
    __syncthreads();  // the queries in LDS, the new record written (read by this task only)
#pragma unroll
    for (int i = 0; i < 32; i++) qv[0][i] = s_q[e][32 * half + i];
  } else {
#pragma unroll
    for (int r = 0; r < M; r++)
#pragma unroll
      for (int i = 0; i < 8; i++) {
        const float4 t = ld4(a.q + (static_cast<size_t>(r) * a.n_heads + 2 * g + e) * 64 + 32 * half + 4 * i);
        qv[r][4 * i] = t.x;
        qv[r][4 * i + 1] = t.y;
        qv[r][4 * i + 2] = t.z;
        qv[r][4 * i + 3] = t.w;
      }
  }
  const float ninf = -__builtin_inff();
  float m[M], dl[M];
  float4 o[M][2];
#pragma unroll
  for (int r = 0; r < M; r++) {
    m[r] = ninf;
    dl[r] = 0.0f;
    o[r][0] = o[r][1] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  }
  // One 16-key slice starting at position b; rec(q) gives key b + q's record
  // and whether it is a prefix record.
  auto slice = [&](int b, auto rec) __attribute__((always_inline)) {
    // Scores.
    const int j = b + kk;
    const auto kr = rec(kk);
    const unsigned char *kp = kr.ptr;
    const bool pre = kr.prefix;
    const int koff = half == 0 ? 0 : (pre ? 32 + 32 * e : 32);
    const int sidx = half == 0 ? 0 : (pre ? 1 + e : 1);
    const uint16_t *ksteps = reinterpret_cast<const uint16_t *>(kp + (pre ? kRecord : kTail) * B);
    const float kstep = bf16_widen(ksteps[sidx]);
    float acc[M];
#pragma unroll
    for (int r = 0; r < M; r++) acc[r] = 0.0f;
#pragma unroll
    for (int w4 = 0; w4 < 2 * B; w4++) {
      const uint4 w = *reinterpret_cast<const uint4 *>(kp + koff * B + 16 * w4);
      const uint32_t words[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
      for (int wi = 0; wi < 4; wi++) {
        constexpr int kPer = 4 / B;  // codes per word
#pragma unroll
        for (int ci = 0; ci < kPer; ci++) {
          float code;
          if constexpr (B == 1)
            code = ci == 0 ? word_code<C, 0>(words[wi]) : ci == 1 ? word_code<C, 1>(words[wi])
                 : ci == 2 ? word_code<C, 2>(words[wi]) : word_code<C, 3>(words[wi]);
          else
            code = ci == 0 ? word_code<C, 0>(words[wi]) : word_code<C, 1>(words[wi]);
          const int d = (16 * w4 + 4 * wi) / B + ci;
#pragma unroll
          for (int r = 0; r < M; r++) acc[r] = fmaf_(qv[r][d], code, acc[r]);
        }
      }
    }
    float p[M], rsv[M];
#pragma unroll
    for (int r = 0; r < M; r++) {
      const float part = acc[r] * kstep;
      const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(part), __float_as_uint(part), false, false);
      float sc = (__uint_as_float(sw[0]) + __uint_as_float(sw[1])) * 0.125f;
      sc = j < vis[r] ? sc : ninf;
      // Slice maximum over the 16 keys (every lane of the row gets it).
      float bm = sc;
      bm = __builtin_fmaxf(bm, dpp<0x128>(bm));
      bm = __builtin_fmaxf(bm, dpp<0x124>(bm));
      bm = __builtin_fmaxf(bm, dpp<0x122>(bm));
      bm = __builtin_fmaxf(bm, dpp<0x121>(bm));
      const float mn = bm > m[r] ? bm : m[r];
      const float rs = m[r] == ninf ? 0.0f : expf_acc(m[r] - mn);
      p[r] = sc == ninf ? 0.0f : prob_exp<FAST>(sc - mn);
      dl[r] = dl[r] * rs + p[r];
      m[r] = mn;
      rsv[r] = rs;
    }
    if (half == 0) {
#pragma unroll
      for (int r = 0; r < M; r++) reinterpret_cast<float *>(&s_p[wave][kk][r])[e] = p[r];
    }
    // Values: rescale, then keys 4i + ks.
#pragma unroll
    for (int r = 0; r < M; r++) {
      const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(rsv[r]), 0));
      const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(rsv[r]), 16));
      if (r0 != 1.0f) o[r][0] = scale4(o[r][0], r0);
      if (r1 != 1.0f) o[r][1] = scale4(o[r][1], r1);
    }
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int q = 4 * i + ks;
      const auto vr = rec(q);
      const unsigned char *vp = vr.ptr;
      const bool vpre = vr.prefix;
      const int voff = vpre ? 96 : 64;
      const int vsidx = (vpre ? 3 : 2) + (dq >> 3);
      const float vstep = bf16_widen(reinterpret_cast<const uint16_t *>(vp + (vpre ? kRecord : kTail) * B)[vsidx]);
      const float4 cv = codes4<C>(vp + (voff + 4 * dq) * B);
#pragma unroll
      for (int r = 0; r < M; r++) {
        const float2 pp = s_p[wave][q][r];
        // A masked or vanished key adds nothing, whatever its step holds.
        const float pv0 = pp.x == 0.0f ? 0.0f : pp.x * vstep;
        const float pv1 = pp.y == 0.0f ? 0.0f : pp.y * vstep;
        o[r][0] = make_float4(fmaf_(pv0, cv.x, o[r][0].x), fmaf_(pv0, cv.y, o[r][0].y), fmaf_(pv0, cv.z, o[r][0].z),
                              fmaf_(pv0, cv.w, o[r][0].w));
        o[r][1] = make_float4(fmaf_(pv1, cv.x, o[r][1].x), fmaf_(pv1, cv.y, o[r][1].y), fmaf_(pv1, cv.z, o[r][1].z),
                              fmaf_(pv1, cv.w, o[r][1].w));
      }
    }
  };
  struct RecRef {
    const unsigned char *ptr;
    bool prefix;
  };
  const int rounds = iters / kWaves;
  auto round = [&](const RoundBuf<C> &cur, RoundBuf<C> &next, int t) __attribute__((always_inline)) {
    __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0): this wave's copies of round t
    __syncthreads();                     // everyone's copies; nobody still reads `next`
    issue(next, t + 1 < rounds ? t + 1 : rounds - 1);
    const int b = key0 + kRoundKeys * t;
    const int bw = b + 16 * wave;
    // As in split_partial_kernel: a round wholly inside the visible prefix is
    // scored from LDS, the others read HBM, each branch consuming its own keys.
    if (b + kRoundKeys <= a.prefix_len && b + kRoundKeys <= limit) {
      const unsigned char *base = reinterpret_cast<const unsigned char *>(cur.chunk) + 16 * wave * rbytes;
      slice(bw, [&](int q) { return RecRef{base + q * rbytes, true}; });
    } else {
      slice(bw, [&](int q) {
        const int jj = bw + q < limit ? bw + q : 0;
        const bool pre = jj < a.prefix_len;
        const unsigned char *ptr =
            pre ? a.records + (static_cast<size_t>(g) * a.prefix_len + jj) * rbytes
                : a.tail + (static_cast<size_t>(g) * a.tail_capacity + (jj - a.prefix_len)) * a.tail_bytes;
        return RecRef{ptr, pre};
      });
    }
  };
  int t = 0;
  for (; t + 2 <= rounds; t += 2) {
    round(rb0, rb1, t);
    round(rb1, rb0, t + 1);
  }
  if (t < rounds) round(rb0, rb1, t);
  __builtin_amdgcn_s_waitcnt(0x0f70);  // the repeated copies land before LDS is reused
  // The wave's state: denominators summed over the slice lanes, outputs over
  // the key quarters.
#pragma unroll
  for (int r = 0; r < M; r++) {
    const float den = row_sum16(dl[r]);
#pragma unroll
    for (int h2 = 0; h2 < 2; h2++) {
      float4 v = o[r][h2];
      auto add_pairs16 = [](float x) {
        const auto sw = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
        return __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
      };
      auto add_pairs32 = [](float x) {
        const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
        return __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
      };
      v = make_float4(add_pairs32(add_pairs16(v.x)), add_pairs32(add_pairs16(v.y)), add_pairs32(add_pairs16(v.z)),
                      add_pairs32(add_pairs16(v.w)));
      if (ks == 0) s_o[wave][h2][r][dq] = v;
    }
    if (lane == 0 || lane == 16) s_md[wave][e][r] = make_float2(m[r], den);
  }
  __syncthreads();
  if (lane < 32) {
    const int lg = lane >> 4, lp = lane & 15;
    const int he = lg;
#pragma unroll
    for (int r = 0; r < M; r++) {
      if (r % kWaves != wave) continue;
      float2 md = s_md[0][he][r];
      float4 accv = s_o[0][he][r][lp];
#pragma unroll
      for (int w = 1; w < kWaves; w++) {
        const float2 md2 = s_md[w][he][r];
        merge(md.x, md.y, accv, md2.x, md2.y, s_o[w][he][r][lp]);
      }
      const size_t slot = (static_cast<size_t>(r) * a.n_heads + 2 * g + he) * a.chunks + c;
      *reinterpret_cast<float4 *>(a.part_o + slot * 64 + 4 * lp) = accv;
      if (lp == 0) *reinterpret_cast<float2 *>(a.part_md + slot * 2) = md;
    }
  }
}

// `fixed` (optional): a caller-provided partial-state buffer of
// `fixed_bytes` used instead of the context scratch (nothing is allocated).
template <typename C, int M, bool ROW = false>
int launch_split(Ctx *ctx, SplitDecArgs a, int rows, bool fast, const float *sinks, float *out, float *fixed,
                 size_t fixed_bytes) {
  // Keys per workgroup task, whole multiples of 64 keys (every wave of the
  // task takes the same number of 16-key iterations), at most kMaxChunks
  // chunks. Each task serves two heads. Up to 32,768 positions: about 512
  // tasks (keys per task rounded to the nearest 64), which halves the
  // partial states the combine reads; beyond: about 1024 tasks (rounded up),
  // whose extra parallelism the longer cold scan needs. Measured one-row
  // decode over Q8 records (cold): 16,384 positions 15.6 us with 512 tasks
  // against 17.0 with 1,024; 65,536 positions 28.1 us with 1,024 tasks
  // against 29.0 with 512; 4,160 positions 12.8 us with 520 tasks against
  // 13.2 with 264.
  const long limit = a.last;
  long per = limit <= 32768 ? (limit * a.n_kv / 512 + 32) / 64 * 64 : ((limit * a.n_kv + 1023) / 1024 + 63) / 64 * 64;
  const long min_per = ((limit + kMaxChunks - 1) / kMaxChunks + 63) / 64 * 64;
  if (per < min_per) per = min_per;
  if (per < 64) per = 64;
  const int iters = static_cast<int>(per / 16);
  a.chunks = static_cast<int>((limit + per - 1) / per);
  a.tasks = a.n_kv * a.chunks;
  const size_t slots = static_cast<size_t>(rows) * a.n_heads * a.chunks;
  const size_t need = slots * 66 * sizeof(float);
  if (fixed) {
    FOCR_REQUIRE(need <= fixed_bytes, FOCR_E_UNSUPPORTED,
                 "split decode needs " + std::to_string(need) + " bytes of partial states; the no-alloc path holds " +
                     std::to_string(fixed_bytes));
    a.part_o = fixed;
  } else {
    int rc = ensure_scratch(ctx, need);
    if (rc != FOCR_OK) return rc;
    a.part_o = static_cast<float *>(ctx->scratch);
  }
  a.part_md = a.part_o + slots * 64;
  if constexpr (M <= 2) {
    if (fast)
      hipLaunchKernelGGL((split_scan_kernel<C, M, true, ROW>), dim3(a.tasks), dim3(64 * kWaves), 0, ctx->stream, a,
                         iters, rows);
    else
      hipLaunchKernelGGL((split_scan_kernel<C, M, false, ROW>), dim3(a.tasks), dim3(64 * kWaves), 0, ctx->stream, a,
                         iters, rows);
  } else {
    static_assert(!ROW, "the fused row step takes one row");
    if (fast)
      hipLaunchKernelGGL((split_partial_kernel<C, M, true>), dim3(a.tasks), dim3(64 * kWaves), 0, ctx->stream, a,
                         iters, rows);
    else
      hipLaunchKernelGGL((split_partial_kernel<C, M, false>), dim3(a.tasks), dim3(64 * kWaves), 0, ctx->stream, a,
                         iters, rows);
  }
  FOCR_HIP_CHECK(hipGetLastError());
  CombineArgs cb;
  cb.part_o = a.part_o;
  cb.part_md = a.part_md;
  cb.sinks = sinks;
  cb.out = out;
  cb.n_heads = a.n_heads;
  cb.chunks = a.chunks;
  hipLaunchKernelGGL(decode_combine_kernel, dim3(static_cast<unsigned>(rows * a.n_heads)), dim3(64 * kWaves), 0,
                     ctx->stream, cb);
  FOCR_HIP_CHECK(hipGetLastError());
  return FOCR_OK;
}

template <typename C>
int launch_split_rows(Ctx *ctx, const SplitDecArgs &a, int rows, bool fast, const float *sinks, float *out,
                      float *fixed, size_t fixed_bytes) {
  switch (rows) {
    case 1: return launch_split<C, 1>(ctx, a, rows, fast, sinks, out, fixed, fixed_bytes);
    case 2: return launch_split<C, 2>(ctx, a, rows, fast, sinks, out, fixed, fixed_bytes);
    case 3: return launch_split<C, 3>(ctx, a, rows, fast, sinks, out, fixed, fixed_bytes);
    case 4: return launch_split<C, 4>(ctx, a, rows, fast, sinks, out, fixed, fixed_bytes);
    case 5: return launch_split<C, 5>(ctx, a, rows, fast, sinks, out, fixed, fixed_bytes);
    case 6: return launch_split<C, 6>(ctx, a, rows, fast, sinks, out, fixed, fixed_bytes);
    case 7: return launch_split<C, 7>(ctx, a, rows, fast, sinks, out, fixed, fixed_bytes);
    default: return launch_split<C, 8>(ctx, a, rows, fast, sinks, out, fixed, fixed_bytes);
  }
}

// The arguments of a decode over `s`, shared by both entry points.
SplitDecArgs split_args(const KvSplit *s, const float *q) {
  SplitDecArgs a;
  a.records = s->records;
  a.tail = s->tail;
  a.q = q;
  a.prefix_len = static_cast<int>(s->prefix_len);
  a.tail_capacity = static_cast<int>(s->capacity - s->prefix_len);
  a.n_heads = s->n_heads;
  a.n_kv = s->n_kv;
  a.record_bytes = static_cast<int>(s->record_bytes);
  a.tail_bytes = static_cast<int>(s->tail_bytes);
  a.last = static_cast<int>(s->prefix_len + s->tail_len);
  a.qkv = a.rope = nullptr;
  a.q_out = nullptr;
  a.tail_w = nullptr;
  return a;
}

}  // namespace
}  // namespace focr

using namespace focr;

extern "C" {

int focr_kv_seal(focr_ctx *handle, int bits, const float *prefix_k, const float *v, size_t prefix_len,
                 size_t capacity, size_t n_heads, size_t n_kv_heads, size_t head_dim, focr_kv_split **out) {
  Ctx *ctx = reinterpret_cast<Ctx *>(handle);
  FOCR_REQUIRE(ctx && prefix_k && v && out, FOCR_E_ARG, "focr_kv_seal: null argument");
  *out = nullptr;
  FOCR_REQUIRE(bits == 8 || bits == 16, FOCR_E_ARG, "focr_kv_seal: bits must be 8 (Kv::Q8) or 16 (Kv::Q16)");
  FOCR_REQUIRE(head_dim == 64 && n_heads == 2 * n_kv_heads && n_kv_heads >= 1 && n_kv_heads <= 8, FOCR_E_SHAPE,
               "split cache requires Falcon 64-wide paired GQA heads");
  FOCR_REQUIRE(prefix_len > 0 && capacity >= prefix_len && capacity < (size_t(1) << 30), FOCR_E_SHAPE,
               "invalid split-prefix capacity");
  FOCR_REQUIRE(prefix_len * n_kv_heads * kRecord / 256 < (size_t(1) << 31), FOCR_E_SHAPE,
               "split prefix too long for one seal launch");
  FOCR_HIP_CHECK(hipSetDevice(ctx->device));
  KvSplit *s = new KvSplit();
  s->bits = bits;
  s->n_heads = static_cast<int>(n_heads);
  s->n_kv = static_cast<int>(n_kv_heads);
  s->prefix_len = prefix_len;
  s->capacity = capacity;
  const size_t cb = bits / 8;
  s->record_bytes = (kRecord * cb + 10 + 15) / 16 * 16;
  s->tail_bytes = (kTail * cb + 8 + 15) / 16 * 16;
  const size_t rec_total = n_kv_heads * prefix_len * s->record_bytes;
  const size_t tail_total = n_kv_heads * (capacity - prefix_len) * s->tail_bytes;
  hipError_t e = hipMalloc(reinterpret_cast<void **>(&s->records), rec_total);
  if (e == hipSuccess && tail_total) e = hipMalloc(reinterpret_cast<void **>(&s->tail), tail_total);
  if (e == hipSuccess) e = hipMalloc(reinterpret_cast<void **>(&s->error), sizeof(uint32_t));
  if (e == hipSuccess) e = hipMemsetAsync(s->error, 0, sizeof(uint32_t), ctx->stream);
  if (e != hipSuccess) {
    focr_kv_free(reinterpret_cast<focr_kv_split *>(s));
    return set_error(FOCR_E_HIP, std::string("focr_kv_seal: ") + hipGetErrorString(e));
  }
  s->device_bytes = rec_total + tail_total;
  SealArgs a{prefix_k, v, s->records, s->error, static_cast<int>(prefix_len), s->n_heads, s->n_kv,
             static_cast<int>(s->record_bytes)};
  const long nrec = static_cast<long>(n_kv_heads) * prefix_len;
  const long pass = (nrec + kSealPer - 1) / kSealPer;
  const dim3 grid(static_cast<unsigned>((pass * kRecord + 255) / 256));
  static_assert(kRecord % 32 == 0 && kTail % 64 == 0, "blocks are whole half-waves");
  if (bits == 8)
    hipLaunchKernelGGL(seal_kernel<int8_t>, grid, dim3(256), 0, ctx->stream, a, pass);
  else
    hipLaunchKernelGGL(seal_kernel<int16_t>, grid, dim3(256), 0, ctx->stream, a, pass);
  uint32_t err = 0;
  e = hipGetLastError();
  if (e == hipSuccess) e = hipMemcpyAsync(&err, s->error, sizeof(err), hipMemcpyDeviceToHost, ctx->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
  if (e != hipSuccess) {
    focr_kv_free(reinterpret_cast<focr_kv_split *>(s));
    return set_error(FOCR_E_HIP, std::string("focr_kv_seal: ") + hipGetErrorString(e));
  }
  if (err) {
    focr_kv_free(reinterpret_cast<focr_kv_split *>(s));
    if (err & kErrPair) return set_error(FOCR_E_VALUE, "temporal keys differ inside GQA pair; refusing illegal sharing");
    if (err & kErrNonFinite) return set_error(FOCR_E_VALUE, "nonfinite or incomplete KV group");
    return set_error(FOCR_E_VALUE, bits == 8 ? "Q8 KV conversion overflow" : "Q16 KV conversion overflow");
  }
  *out = reinterpret_cast<focr_kv_split *>(s);
  return FOCR_OK;
}

int focr_kv_append(focr_ctx *handle, focr_kv_split *kv, const float *k, const float *v, size_t rows) {
  Ctx *ctx = reinterpret_cast<Ctx *>(handle);
  KvSplit *s = reinterpret_cast<KvSplit *>(kv);
  FOCR_REQUIRE(ctx && s && k && v, FOCR_E_ARG, "focr_kv_append: null argument");
  if (rows == 0) return FOCR_OK;
  FOCR_REQUIRE(s->prefix_len + s->tail_len + rows <= s->capacity, FOCR_E_SHAPE, "split tail capacity");
  FOCR_HIP_CHECK(hipSetDevice(ctx->device));
  AppendArgs a{k, v, s->tail, s->n_kv, static_cast<int>(s->capacity - s->prefix_len), static_cast<int>(s->tail_len),
               static_cast<int>(rows), static_cast<int>(s->tail_bytes)};
  const int threads = static_cast<int>(rows) * s->n_kv * kTail;
  if (s->bits == 8)
    hipLaunchKernelGGL(append_kernel<int8_t>, dim3((threads + 255) / 256), dim3(256), 0, ctx->stream, a);
  else
    hipLaunchKernelGGL(append_kernel<int16_t>, dim3((threads + 255) / 256), dim3(256), 0, ctx->stream, a);
  FOCR_HIP_CHECK(hipGetLastError());
  s->tail_len += rows;
  return FOCR_OK;
}

int focr_kv_qkv_rows(focr_ctx *handle, focr_kv_split *kv, const float *qkv, size_t rows, const float *rope,
                     float *q) {
  Ctx *ctx = reinterpret_cast<Ctx *>(handle);
  KvSplit *s = reinterpret_cast<KvSplit *>(kv);
  FOCR_REQUIRE(ctx && s && qkv && rope && q, FOCR_E_ARG, "focr_kv_qkv_rows: null argument");
  if (rows == 0) return FOCR_OK;
  FOCR_REQUIRE(rows <= 8, FOCR_E_SHAPE, "decode takes 1..=8 rows");
  FOCR_REQUIRE(s->prefix_len + s->tail_len + rows <= s->capacity, FOCR_E_SHAPE, "split tail capacity");
  FOCR_HIP_CHECK(hipSetDevice(ctx->device));
  RowAppendArgs a{qkv, rope, q, s->tail, s->n_heads, s->n_kv, static_cast<int>(s->capacity - s->prefix_len),
                  static_cast<int>(s->tail_len), static_cast<int>(s->tail_bytes)};
  if (s->bits == 8)
    hipLaunchKernelGGL(row_append_kernel<int8_t>, dim3(static_cast<unsigned>(rows)), dim3(64 * kRowWaves), 0,
                       ctx->stream, a);
  else
    hipLaunchKernelGGL(row_append_kernel<int16_t>, dim3(static_cast<unsigned>(rows)), dim3(64 * kRowWaves), 0,
                       ctx->stream, a);
  FOCR_HIP_CHECK(hipGetLastError());
  s->tail_len += rows;
  return FOCR_OK;
}

int focr_kv_decode_row(focr_ctx *handle, focr_kv_split *kv, const float *qkv, const float *rope, const float *sinks,
                       float *q, float *out) {
  Ctx *ctx = reinterpret_cast<Ctx *>(handle);
  KvSplit *s = reinterpret_cast<KvSplit *>(kv);
  FOCR_REQUIRE(ctx && s && qkv && rope && sinks && out, FOCR_E_ARG, "focr_kv_decode_row: null argument");
  FOCR_REQUIRE(s->prefix_len + s->tail_len + 1 <= s->capacity, FOCR_E_SHAPE, "split tail capacity");
  FOCR_REQUIRE(s->n_heads == 2 * s->n_kv, FOCR_E_SHAPE, "split decode: two query heads per KV head");
  FOCR_HIP_CHECK(hipSetDevice(ctx->device));
  SplitDecArgs a = split_args(s, nullptr);
  a.last += 1;  // the new row is position prefix_len + tail_len
  a.qkv = qkv;
  a.rope = rope;
  a.q_out = q;
  a.tail_w = s->tail + s->tail_len * s->tail_bytes;
  const int rc = s->bits == 8 ? launch_split<int8_t, 1, true>(ctx, a, 1, s->fast_exp, sinks, out, nullptr, 0)
                              : launch_split<int16_t, 1, true>(ctx, a, 1, s->fast_exp, sinks, out, nullptr, 0);
  if (rc == FOCR_OK) s->tail_len += 1;
  return rc;
}

int focr_kv_attention_decode(focr_ctx *handle, const focr_kv_split *kv, const float *q, size_t rows,
                             const float *sinks, float *out) {
  Ctx *ctx = reinterpret_cast<Ctx *>(handle);
  const KvSplit *s = reinterpret_cast<const KvSplit *>(kv);
  FOCR_REQUIRE(ctx && s && q && sinks && out, FOCR_E_ARG, "focr_kv_attention_decode: null argument");
  FOCR_REQUIRE(rows >= 1 && rows <= 8 && rows <= (s->tail_len > 0 ? s->tail_len : 1), FOCR_E_SHAPE,
               "split decode: 1 to 8 rows, at most the appended positions");
  FOCR_HIP_CHECK(hipSetDevice(ctx->device));
  const SplitDecArgs a = split_args(s, q);
  const int r = static_cast<int>(rows);
  return s->bits == 8 ? launch_split_rows<int8_t>(ctx, a, r, s->fast_exp, sinks, out, nullptr, 0)
                      : launch_split_rows<int16_t>(ctx, a, r, s->fast_exp, sinks, out, nullptr, 0);
}

int focr_kv_attention_decode_noalloc(focr_ctx *handle, const focr_kv_split *kv, const float *q, size_t rows,
                                     const float *sinks, float *out) {
  Ctx *ctx = reinterpret_cast<Ctx *>(handle);
  const KvSplit *s = reinterpret_cast<const KvSplit *>(kv);
  FOCR_REQUIRE(ctx && s && q && sinks && out, FOCR_E_ARG, "focr_kv_attention_decode_noalloc: null argument");
  FOCR_REQUIRE(rows >= 1 && rows <= 8 && rows <= (s->tail_len > 0 ? s->tail_len : 1), FOCR_E_SHAPE,
               "split decode: 1 to 8 rows, at most the appended positions");
  FOCR_HIP_CHECK(hipSetDevice(ctx->device));
  float *fixed = noalloc_scratch(ctx->device);
  FOCR_REQUIRE(fixed, FOCR_E_HIP, "the no-alloc scratch of this device was not resolved (focr_ctx_create does it)");
  const SplitDecArgs a = split_args(s, q);
  const int r = static_cast<int>(rows);
  return s->bits == 8 ? launch_split_rows<int8_t>(ctx, a, r, s->fast_exp, sinks, out, fixed, kNoAllocScratchBytes)
                      : launch_split_rows<int16_t>(ctx, a, r, s->fast_exp, sinks, out, fixed, kNoAllocScratchBytes);
}

int focr_kv_dequantize(focr_ctx *handle, const focr_kv_split *kv, float *prefix_k, float *values, float *generated_k) {
  Ctx *ctx = reinterpret_cast<Ctx *>(handle);
  const KvSplit *s = reinterpret_cast<const KvSplit *>(kv);
  FOCR_REQUIRE(ctx && s && prefix_k && values && (generated_k || s->tail_len == 0), FOCR_E_ARG,
               "focr_kv_dequantize: null argument");
  FOCR_HIP_CHECK(hipSetDevice(ctx->device));
  DequantArgs a{s->records, s->tail, prefix_k, values, generated_k, static_cast<int>(s->prefix_len),
                static_cast<int>(s->tail_len), static_cast<int>(s->capacity - s->prefix_len), s->n_heads, s->n_kv,
                static_cast<int>(s->record_bytes), static_cast<int>(s->tail_bytes)};
  const long items = static_cast<long>(s->prefix_len) * s->n_kv * kRecord + static_cast<long>(s->tail_len) * s->n_kv * kTail;
  const dim3 grid(static_cast<unsigned>((items + 255) / 256));
  if (s->bits == 8)
    hipLaunchKernelGGL(dequantize_kernel<int8_t>, grid, dim3(256), 0, ctx->stream, a);
  else
    hipLaunchKernelGGL(dequantize_kernel<int16_t>, grid, dim3(256), 0, ctx->stream, a);
  FOCR_HIP_CHECK(hipGetLastError());
  return FOCR_OK;
}

int focr_kv_truncate_tail(focr_kv_split *kv, size_t tail_len) {
  KvSplit *s = reinterpret_cast<KvSplit *>(kv);
  FOCR_REQUIRE(s, FOCR_E_ARG, "focr_kv_truncate_tail: null cache");
  FOCR_REQUIRE(tail_len <= s->tail_len, FOCR_E_SHAPE, "cannot grow the tail by truncation");
  s->tail_len = tail_len;
  return FOCR_OK;
}

int focr_kv_info(const focr_kv_split *kv, int *bits, size_t *prefix_len, size_t *tail_len, size_t *capacity,
                 size_t *device_bytes) {
  const KvSplit *s = reinterpret_cast<const KvSplit *>(kv);
  FOCR_REQUIRE(s, FOCR_E_ARG, "focr_kv_info: null cache");
  if (bits) *bits = s->bits;
  if (prefix_len) *prefix_len = s->prefix_len;
  if (tail_len) *tail_len = s->tail_len;
  if (capacity) *capacity = s->capacity;
  if (device_bytes) *device_bytes = s->device_bytes;
  return FOCR_OK;
}

int focr_kv_set_fast_exp(focr_kv_split *kv, int fast) {
  KvSplit *s = reinterpret_cast<KvSplit *>(kv);
  FOCR_REQUIRE(s, FOCR_E_ARG, "focr_kv_set_fast_exp: null cache");
  s->fast_exp = fast != 0;
  return FOCR_OK;
}

int focr_kv_fast_exp(const focr_kv_split *kv, int *fast) {
  const KvSplit *s = reinterpret_cast<const KvSplit *>(kv);
  FOCR_REQUIRE(s && fast, FOCR_E_ARG, "focr_kv_fast_exp: null argument");
  *fast = s->fast_exp ? 1 : 0;
  return FOCR_OK;
}

int focr_kv_free(focr_kv_split *kv) {
  KvSplit *s = reinterpret_cast<KvSplit *>(kv);
  if (!s) return FOCR_OK;
  if (s->records) (void)hipFree(s->records);
  if (s->tail) (void)hipFree(s->tail);
  if (s->error) (void)hipFree(s->error);
  delete s;
  return FOCR_OK;
}

}  // extern "C"
