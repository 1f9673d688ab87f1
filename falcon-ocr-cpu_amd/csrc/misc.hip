// Element-wise and per-row kernels of the hot path: weight dequantization
// (A1), RMS row scales (A6) and greedy argmax (A9). All HBM-bound.
#include "focr_internal.hpp"
#include "rms_tree.hpp"

namespace focr {
namespace {

// dequantize_row for every row (src/quant/linear.rs:246-262, dot.rs:25-29):
// w = fl(code * scale), exception columns replaced by their FP32 weights.
template <typename T>
__global__ __launch_bounds__(256) void dequantize_kernel(const T *__restrict__ codes, const float *__restrict__ scales,
                                                         const int16_t *__restrict__ exc_index,
                                                         const float *__restrict__ exc_vals, int n_exc, size_t n,
                                                         size_t k, size_t group, size_t groups, float *__restrict__ out) {
  const size_t total = n * k;
  for (size_t i = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x; i < total;
       i += static_cast<size_t>(gridDim.x) * blockDim.x) {
    const size_t row = i / k, col = i % k;
    float w = static_cast<float>(static_cast<int32_t>(codes[i])) * scales[row * groups + col / group];
    if (exc_index) {
      const int e = exc_index[col];
      if (e >= 0) w = exc_vals[row * n_exc + e];
    }
    out[i] = w;
  }
}

// The same, four consecutive weights of a row per thread (k and the group a
// multiple of 4, fewer than 2^31 weights): 32-bit indexing, one code load,
// one scale, one 16-byte store.
template <typename T>
__global__ __launch_bounds__(256) void dequantize4_kernel(const T *__restrict__ codes, const float *__restrict__ scales,
                                                          const int16_t *__restrict__ exc_index,
                                                          const float *__restrict__ exc_vals, int n_exc, int n, int k,
                                                          int group, int groups, float *__restrict__ out) {
  const int per_row = k / 4, quads = n * per_row;
  for (int q = blockIdx.x * 256 + threadIdx.x; q < quads; q += gridDim.x * 256) {
    const int row = q / per_row, col = (q - row * per_row) * 4;
    const float sc = scales[static_cast<size_t>(row) * groups + col / group];
    float w[4];
    if constexpr (sizeof(T) == 2) {
      const uint2 u = *reinterpret_cast<const uint2 *>(codes + static_cast<size_t>(q) * 4);
      w[0] = static_cast<float>(static_cast<int16_t>(u.x & 0xffffu));
      w[1] = static_cast<float>(static_cast<int16_t>(u.x >> 16));
      w[2] = static_cast<float>(static_cast<int16_t>(u.y & 0xffffu));
      w[3] = static_cast<float>(static_cast<int16_t>(u.y >> 16));
    } else {
      const uint32_t u = *reinterpret_cast<const uint32_t *>(codes + static_cast<size_t>(q) * 4);
#pragma unroll
      for (int i = 0; i < 4; i++) w[i] = static_cast<float>(static_cast<int8_t>((u >> (8 * i)) & 0xffu));
    }
#pragma unroll
    for (int i = 0; i < 4; i++) w[i] = w[i] * sc;
    if (exc_index) {
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int e = exc_index[col + i];
        if (e >= 0) w[i] = exc_vals[static_cast<size_t>(row) * n_exc + e];
      }
    }
    *reinterpret_cast<float4 *>(out + static_cast<size_t>(q) * 4) = make_float4(w[0], w[1], w[2], w[3]);
  }
}

// One 32-element leaf of sum_squares_pairwise (src/kernels/mod.rs:546-552):
// squares into 32 zero-padded slots, then partial[i] += partial[i + w] for
// w = 16, 8, 4, 2, 1.
__device__ float leaf_sum(const float *x, int len) {
  float part[32];
#pragma unroll
  for (int i = 0; i < 32; i++) part[i] = i < len ? x[i] * x[i] : 0.0f;
#pragma unroll
  for (int w = 16; w >= 1; w /= 2)
#pragma unroll
    for (int i = 0; i < w; i++) part[i] = part[i] + part[i + w];
  return part[0];
}

__device__ __forceinline__ int split_point(int len) { return ((len / 2 + 31) / 32) * 32; }

constexpr int kMaxLeaves = 1024;  // widths up to 16384 (leaves <= 2 * width / 32)

// rms_scale (src/kernels/mod.rs:531-553): one wave per row. Lane 0 walks the
// recursive halving tree (split at (len/2).next_multiple_of(32)) to list the
// leaves left to right, the wave sums the leaves in parallel, and lane 0
// adds them back up the same tree: left + right at every node.
__global__ __launch_bounds__(64) void row_scales_kernel(const float *__restrict__ h, int width, float eps,
                                                        float *__restrict__ out) {
  __shared__ int leaf_start[kMaxLeaves];
  __shared__ int leaf_len[kMaxLeaves];
  __shared__ float leaf_val[kMaxLeaves];
  __shared__ int leaf_count;
  const float *row = h + static_cast<size_t>(blockIdx.x) * width;
  if (threadIdx.x == 0) {
    int stack_start[40], stack_len[40], sp = 0, count = 0;
    stack_start[sp] = 0;
    stack_len[sp++] = width;
    while (sp > 0) {
      const int s = stack_start[--sp], len = stack_len[sp];
      if (len > 32) {
        const int m = split_point(len);
        stack_start[sp] = s + m;  // right, visited after left
        stack_len[sp++] = len - m;
        stack_start[sp] = s;
        stack_len[sp++] = m;
      } else {
        leaf_start[count] = s;
        leaf_len[count++] = len;
      }
    }
    leaf_count = count;
  }
  __syncthreads();
  for (int i = threadIdx.x; i < leaf_count; i += 64) leaf_val[i] = leaf_sum(row + leaf_start[i], leaf_len[i]);
  __syncthreads();
  if (threadIdx.x != 0) return;
  // Post-order evaluation: frame state 0 = descend left, 1 = descend right, 2 = add.
  int f_len[40], f_state[40], sp = 0, next_leaf = 0;
  float f_left[40], ret = 0.0f;
  f_len[0] = width;
  f_state[0] = 0;
  sp = 1;
  while (sp > 0) {
    const int top = sp - 1, len = f_len[top];
    if (len <= 32) {
      ret = leaf_val[next_leaf++];
      sp--;
      continue;
    }
    const int m = split_point(len);
    if (f_state[top] == 0) {
      f_state[top] = 1;
      f_len[sp] = m;
      f_state[sp++] = 0;
    } else if (f_state[top] == 1) {
      f_left[top] = ret;
      f_state[top] = 2;
      f_len[sp] = len - m;
      f_state[sp++] = 0;
    } else {
      ret = f_left[top] + ret;
      sp--;
    }
  }
  // (sum / width + eps).sqrt().recip(): IEEE division and square root.
  out[blockIdx.x] = __fdiv_rn(1.0f, __builtin_sqrtf(__fdiv_rn(ret, static_cast<float>(width)) + eps));
}

// rms_scale for the model's widths: one wave per row, leaves in parallel and
// the reference's addition order unrolled at compile time (rms_tree.hpp).
template <int LEN>
__global__ __launch_bounds__(256) void row_scales_fixed_kernel(const float *__restrict__ h, int rows, float eps,
                                                               float *__restrict__ out) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const float *x = h + static_cast<size_t>(row) * LEN;
  const float scale = rms_scale_wave<LEN>([&](int i) { return x[i]; }, eps);
  if ((threadIdx.x & 63) == 0) out[row] = scale;
}

// argmax (src/runner/mod.rs:916-930): first index of the maximum, and a flag
// when any value is non-finite. One workgroup of 1024 threads per row; each
// thread keeps the first maximum of its own values (visited in ascending
// index order), and the workgroup combines (value, index) pairs, the smaller
// index winning ties. Every thread issues its loads of a pass (8 float4, or 8
// floats for rows that are not 16-byte aligned) before comparing them.
__global__ __launch_bounds__(1024) void argmax_kernel(const float *__restrict__ logits, int vocab,
                                                      uint32_t *__restrict__ result) {
  const float *row = logits + static_cast<size_t>(blockIdx.x) * vocab;
  const int tid = threadIdx.x;
  float best = -__builtin_inff();
  int best_i = -1;
  int nonfinite = 0;
  auto visit = [&](float v, int i) {
    nonfinite |= !__builtin_isfinite(v);
    if (best_i < 0 || v > best) {
      best = v;
      best_i = i;
    }
  };
  const bool vec = (reinterpret_cast<uintptr_t>(row) & 15) == 0;
  if (vec) {
    const int quads = vocab / 4;
    for (int base = 0; base < quads; base += 8 * 1024) {
      float4 q[8];
#pragma unroll
      for (int j = 0; j < 8; j++) {
        const int at = base + 1024 * j + tid;
        q[j] = at < quads ? reinterpret_cast<const float4 *>(row)[at] : make_float4(0.f, 0.f, 0.f, 0.f);
      }
#pragma unroll
      for (int j = 0; j < 8; j++) {
        const int at = base + 1024 * j + tid;
        if (at < quads) {
          visit(q[j].x, 4 * at);
          visit(q[j].y, 4 * at + 1);
          visit(q[j].z, 4 * at + 2);
          visit(q[j].w, 4 * at + 3);
        }
      }
    }
    for (int i = 4 * quads + tid; i < vocab; i += 1024) visit(row[i], i);
  } else {
    for (int base = 0; base < vocab; base += 8 * 1024) {
      float v[8];
#pragma unroll
      for (int j = 0; j < 8; j++) {
        const int at = base + 1024 * j + tid;
        v[j] = at < vocab ? row[at] : 0.0f;
      }
#pragma unroll
      for (int j = 0; j < 8; j++) {
        const int at = base + 1024 * j + tid;
        if (at < vocab) visit(v[j], at);
      }
    }
  }
  // Wave, then workgroup combination.
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const float ov = __shfl_xor(best, off);
    const int oi = __shfl_xor(best_i, off);
    if (oi >= 0 && (best_i < 0 || ov > best || (ov == best && oi < best_i))) {
      best = ov;
      best_i = oi;
    }
    nonfinite |= __shfl_xor(nonfinite, off);
  }
  __shared__ float s_val[16];
  __shared__ int s_idx[16];
  __shared__ int s_bad[16];
  if ((tid & 63) == 0) {
    s_val[tid >> 6] = best;
    s_idx[tid >> 6] = best_i;
    s_bad[tid >> 6] = nonfinite;
  }
  __syncthreads();
  if (tid == 0) {
    float fv = s_val[0];
    int fi = s_idx[0], bad = s_bad[0];
    for (int w = 1; w < 16; w++) {
      bad |= s_bad[w];
      if (s_idx[w] >= 0 && (fi < 0 || s_val[w] > fv || (s_val[w] == fv && s_idx[w] < fi))) {
        fv = s_val[w];
        fi = s_idx[w];
      }
    }
    result[2 * blockIdx.x] = static_cast<uint32_t>(fi);
    result[2 * blockIdx.x + 1] = static_cast<uint32_t>(bad);
  }
}

}  // namespace

int launch_dequantize(Ctx *ctx, const Linear *lin, float *out) {
  FOCR_HIP_CHECK(hipSetDevice(ctx->device));
  const size_t total = lin->n * lin->k;
  if (lin->bits == 32) {
    FOCR_HIP_CHECK(hipMemcpyAsync(out, lin->codes, total * sizeof(float), hipMemcpyDeviceToDevice, ctx->stream));
    return FOCR_OK;
  }
  if (lin->k % 4 == 0 && lin->group % 4 == 0 && total < (size_t(1) << 31) &&
      reinterpret_cast<uintptr_t>(out) % 16 == 0) {
    const size_t want = (total / 4 + 255) / 256;
    const int blocks = static_cast<int>(want < 65536 ? want : 65536);
    const int n = static_cast<int>(lin->n), k = static_cast<int>(lin->k), group = static_cast<int>(lin->group),
              groups = static_cast<int>(lin->groups), n_exc = static_cast<int>(lin->n_exc);
    if (lin->bits == 8)
      hipLaunchKernelGGL(dequantize4_kernel<int8_t>, dim3(blocks), dim3(256), 0, ctx->stream,
                         static_cast<const int8_t *>(lin->codes), lin->scales, lin->exc_index, lin->exc_vals, n_exc, n,
                         k, group, groups, out);
    else
      hipLaunchKernelGGL(dequantize4_kernel<int16_t>, dim3(blocks), dim3(256), 0, ctx->stream,
                         static_cast<const int16_t *>(lin->codes), lin->scales, lin->exc_index, lin->exc_vals, n_exc,
                         n, k, group, groups, out);
    FOCR_HIP_CHECK(hipGetLastError());
    return FOCR_OK;
  }
  const size_t want = (total + 255) / 256;
  const int blocks = static_cast<int>(want < 65536 ? want : 65536);
  if (lin->bits == 8)
    hipLaunchKernelGGL(dequantize_kernel<int8_t>, dim3(blocks), dim3(256), 0, ctx->stream,
                       static_cast<const int8_t *>(lin->codes), lin->scales, lin->exc_index, lin->exc_vals,
                       static_cast<int>(lin->n_exc), lin->n, lin->k, lin->group, lin->groups, out);
  else
    hipLaunchKernelGGL(dequantize_kernel<int16_t>, dim3(blocks), dim3(256), 0, ctx->stream,
                       static_cast<const int16_t *>(lin->codes), lin->scales, lin->exc_index, lin->exc_vals,
                       static_cast<int>(lin->n_exc), lin->n, lin->k, lin->group, lin->groups, out);
  FOCR_HIP_CHECK(hipGetLastError());
  return FOCR_OK;
}

int launch_row_scales(Ctx *ctx, const float *h, size_t rows, size_t width, float eps, float *out) {
  FOCR_REQUIRE(width <= 16384, FOCR_E_SHAPE, "focr_row_scales: width above 16384");
  FOCR_REQUIRE(rows < (size_t(1) << 31), FOCR_E_SHAPE, "focr_row_scales: too many rows");
  FOCR_HIP_CHECK(hipSetDevice(ctx->device));
  const dim3 grid(static_cast<unsigned>((rows + 3) / 4)), block(256);
  const int r = static_cast<int>(rows);
  switch (width) {
    case 64: hipLaunchKernelGGL(row_scales_fixed_kernel<64>, grid, block, 0, ctx->stream, h, r, eps, out); break;
    case 768: hipLaunchKernelGGL(row_scales_fixed_kernel<768>, grid, block, 0, ctx->stream, h, r, eps, out); break;
    case 1024: hipLaunchKernelGGL(row_scales_fixed_kernel<1024>, grid, block, 0, ctx->stream, h, r, eps, out); break;
    case 2304: hipLaunchKernelGGL(row_scales_fixed_kernel<2304>, grid, block, 0, ctx->stream, h, r, eps, out); break;
    case 4096: hipLaunchKernelGGL(row_scales_fixed_kernel<4096>, grid, block, 0, ctx->stream, h, r, eps, out); break;
    default:
      // Any other width: lane 0 walks the tree.
      hipLaunchKernelGGL(row_scales_kernel, dim3(static_cast<unsigned>(rows)), dim3(64), 0, ctx->stream, h,
                         static_cast<int>(width), eps, out);
  }
  FOCR_HIP_CHECK(hipGetLastError());
  return FOCR_OK;
}

int launch_argmax(Ctx *ctx, const float *logits, size_t rows, size_t vocab, uint32_t *result_dev) {
  FOCR_REQUIRE(rows < (size_t(1) << 31), FOCR_E_SHAPE, "focr_argmax: too many rows");
  hipLaunchKernelGGL(argmax_kernel, dim3(static_cast<unsigned>(rows)), dim3(1024), 0, ctx->stream, logits,
                     static_cast<int>(vocab), result_dev);
  FOCR_HIP_CHECK(hipGetLastError());
  return FOCR_OK;
}

}  // namespace focr
