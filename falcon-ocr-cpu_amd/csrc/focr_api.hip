// The C ABI (include/focr_hip.h): contexts, error reporting, device memory,
// matrix upload with the device layouts the kernels read, and dispatch.
#include <algorithm>
#include <cmath>
#include <cstring>
#include <new>
#include <vector>

#include "focr_internal.hpp"

namespace focr {

namespace {
thread_local std::string g_last_error;
}

int set_error(int code, const std::string &message) {
  g_last_error = message;
  return code;
}

int ensure_scratch(Ctx *ctx, size_t bytes) {
  if (bytes <= ctx->scratch_bytes) return FOCR_OK;
  // Growing frees the old buffer: a graph captured earlier would replay into
  // freed memory, and neither a free nor a synchronization may run while the
  // stream is being captured. Callers that capture pre-grow the scratch with
  // focr_ctx_reserve_scratch (or one uncaptured call of the same shape).
  hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
  FOCR_HIP_CHECK(hipStreamIsCapturing(ctx->stream, &capture));
  FOCR_REQUIRE(capture == hipStreamCaptureStatusNone, FOCR_E_UNSUPPORTED,
               "the context scratch must grow to " + std::to_string(bytes) +
                   " bytes, which cannot happen during stream capture; call focr_ctx_reserve_scratch first");
  if (ctx->scratch) {
    FOCR_HIP_CHECK(hipStreamSynchronize(ctx->stream));
    FOCR_HIP_CHECK(hipFree(ctx->scratch));
    ctx->scratch = nullptr;
    ctx->scratch_bytes = 0;
  }
  size_t grown = std::max(bytes, static_cast<size_t>(1) << 20);
  FOCR_HIP_CHECK(hipMalloc(&ctx->scratch, grown));
  ctx->scratch_bytes = grown;
  return FOCR_OK;
}

// The context's work moves to a new stream only behind everything already
// queued on the old one (an event the new stream waits for), so a call on the
// new stream cannot overwrite the context scratch while an earlier call on
// the old stream still reads it. A stream under capture cannot wait for an
// event recorded outside the capture: when either stream is being captured
// the switch happens without the wait, and the caller orders the two streams
// (as torch.cuda.graph's side stream is ordered by wait_stream first).
int order_streams(Ctx *ctx, hipStream_t from, hipStream_t to) {
  if (from == to) return FOCR_OK;
  hipStreamCaptureStatus cap_to = hipStreamCaptureStatusNone, cap_from = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(to, &cap_to) != hipSuccess || cap_to != hipStreamCaptureStatusNone ||
      hipStreamIsCapturing(from, &cap_from) != hipSuccess || cap_from != hipStreamCaptureStatusNone) {
    // A refused query (the null stream while another stream captures)
    // leaves no error behind for the next launch check.
    (void)hipGetLastError();
    return FOCR_OK;
  }
  FOCR_HIP_CHECK(hipEventRecord(ctx->order, from));
  FOCR_HIP_CHECK(hipStreamWaitEvent(to, ctx->order, 0));
  return FOCR_OK;
}

namespace {

int code_bytes(int bits) { return bits == 8 ? 1 : bits == 16 ? 2 : 4; }

// Copies a host vector to a new device buffer.
template <typename T>
int upload_vector(const std::vector<T> &host, T **dev, size_t *total) {
  if (host.empty()) {
    *dev = nullptr;
    return FOCR_OK;
  }
  size_t bytes = host.size() * sizeof(T);
  FOCR_HIP_CHECK(hipMalloc(reinterpret_cast<void **>(dev), bytes));
  FOCR_HIP_CHECK(hipMemcpy(*dev, host.data(), bytes, hipMemcpyHostToDevice));
  *total += bytes;
  return FOCR_OK;
}

void free_linear(Linear *lin) {
  void *ptrs[] = {lin->codes,     lin->scales,      lin->exc_cols, lin->exc_vals,
                  lin->exc_index, lin->gemv_codes,  lin->gemv_scales,
                  lin->i16_b,     lin->i16_wsum,    lin->i16_sw,   lin->pair_w,
                  lin->pair_wexp};
  for (void *p : ptrs)
    if (p) (void)hipFree(p);
}

// The decode GEMV tiles (see Linear in focr_internal.hpp).
template <typename T>
void build_gemv_tiles(const Linear &lin, const T *codes, const float *scales,
                      std::vector<uint8_t> &tiled, std::vector<float> &tiled_scales) {
  const size_t B = sizeof(T);
  const size_t S = 16 / (2 * B);  // blocks per step
  const size_t nb = lin.k / 32;
  const size_t steps = lin.gemv_steps, tiles = lin.gemv_tiles, sps = lin.gemv_sps;
  tiled.assign(tiles * steps * 64 * 16, 0);
  if (sps) tiled_scales.assign(tiles * steps * 2 * 2 * sps, 0.0f);
  for (size_t tile = 0; tile < tiles; tile++)
    for (size_t step = 0; step < steps; step++) {
      uint8_t *chunk = tiled.data() + (tile * steps + step) * 64 * 16;
      for (size_t lane = 0; lane < 64; lane++) {
        const size_t h = lane / 32, p = lane % 32;
        for (size_t s = 0; s < S; s++)
          for (size_t c = 0; c < 2; c++) {
            const size_t b = step * S + s, ch = tile * kGemvChannels + h * 2 + c;
            T value = T(0);
            if (b < nb && ch < lin.n) value = codes[ch * lin.k + 32 * b + p];
            std::memcpy(chunk + lane * 16 + (s * 2 + c) * B, &value, B);
          }
      }
      if (sps)
        for (size_t h = 0; h < 2; h++)
          for (size_t c = 0; c < 2; c++)
            for (size_t g = 0; g < sps; g++) {
              const size_t ch = tile * kGemvChannels + h * 2 + c;
              const size_t block = step * S + g * (lin.group / 32);
              float value = 0.0f;
              if (ch < lin.n && block < nb) value = scales[ch * lin.groups + (32 * block) / lin.group];
              tiled_scales[(((tile * steps + step) * 2 + h) * 2 + c) * sps + g] = value;
            }
    }
}

}  // namespace
}  // namespace focr

using namespace focr;

extern "C" {

const char *focr_last_error(void) { return g_last_error.c_str(); }

int focr_ctx_create(int device, focr_ctx **out) {
  FOCR_REQUIRE(out, FOCR_E_ARG, "focr_ctx_create: null output");
  int count = 0;
  FOCR_HIP_CHECK(hipGetDeviceCount(&count));
  FOCR_REQUIRE(device >= 0 && device < count, FOCR_E_ARG, "focr_ctx_create: no such device");
  FOCR_HIP_CHECK(hipSetDevice(device));
  hipDeviceProp_t prop;
  FOCR_HIP_CHECK(hipGetDeviceProperties(&prop, device));
  FOCR_REQUIRE(std::strncmp(prop.gcnArchName, "gfx950", 6) == 0, FOCR_E_UNSUPPORTED,
               std::string("focr_hip is built for gfx950, device is ") + prop.gcnArchName);
  int rc = noalloc_scratch_init(device);
  if (rc != FOCR_OK) return rc;
  Ctx *ctx = new (std::nothrow) Ctx();
  FOCR_REQUIRE(ctx, FOCR_E_ARG, "focr_ctx_create: out of host memory");
  ctx->device = device;
  hipError_t err = hipStreamCreateWithFlags(&ctx->own, hipStreamNonBlocking);
  if (err != hipSuccess) {
    delete ctx;
    return set_error(FOCR_E_HIP, std::string("hipStreamCreate: ") + hipGetErrorString(err));
  }
  ctx->stream = ctx->own;
  err = hipEventCreateWithFlags(&ctx->order, hipEventDisableTiming);
  if (err != hipSuccess) {
    (void)hipStreamDestroy(ctx->own);
    delete ctx;
    return set_error(FOCR_E_HIP, std::string("hipEventCreate: ") + hipGetErrorString(err));
  }
  err = hipMalloc(&ctx->rms_dev, 8 * sizeof(float));
  if (err != hipSuccess) {
    (void)hipEventDestroy(ctx->order);
    (void)hipStreamDestroy(ctx->own);
    delete ctx;
    return set_error(FOCR_E_HIP, std::string("hipMalloc: ") + hipGetErrorString(err));
  }
  *out = reinterpret_cast<focr_ctx *>(ctx);
  return FOCR_OK;
}

int focr_ctx_destroy(focr_ctx *handle) {
  Ctx *ctx = reinterpret_cast<Ctx *>(handle);
  if (!ctx) return FOCR_OK;
  FOCR_HIP_CHECK(hipSetDevice(ctx->device));
  FOCR_HIP_CHECK(hipStreamSynchronize(ctx->stream));
  if (ctx->scratch) FOCR_HIP_CHECK(hipFree(ctx->scratch));
  if (ctx->argmax_dev) FOCR_HIP_CHECK(hipFree(ctx->argmax_dev));
  if (ctx->rms_dev) FOCR_HIP_CHECK(hipFree(ctx->rms_dev));
  FOCR_HIP_CHECK(hipEventDestroy(ctx->order));
  FOCR_HIP_CHECK(hipStreamDestroy(ctx->own));
  delete ctx;
  return FOCR_OK;
}

int focr_ctx_set_stream(focr_ctx *handle, void *stream) {
  Ctx *ctx = reinterpret_cast<Ctx *>(handle);
  FOCR_REQUIRE(ctx, FOCR_E_ARG, "focr_ctx_set_stream: null context");
  const int rc = order_streams(ctx, ctx->stream, static_cast<hipStream_t>(stream));
  if (rc != FOCR_OK) return rc;
  ctx->stream = static_cast<hipStream_t>(stream);
  return FOCR_OK;
}

int focr_ctx_use_own_stream(focr_ctx *handle) {
  Ctx *ctx = reinterpret_cast<Ctx *>(handle);
  FOCR_REQUIRE(ctx, FOCR_E_ARG, "focr_ctx_use_own_stream: null context");
  const int rc = order_streams(ctx, ctx->stream, ctx->own);
  if (rc != FOCR_OK) return rc;
  ctx->stream = ctx->own;
  return FOCR_OK;
}

void *focr_ctx_stream(const focr_ctx *handle) {
  const Ctx *ctx = reinterpret_cast<const Ctx *>(handle);
  return ctx ? static_cast<void *>(ctx->stream) : nullptr;
}

int focr_ctx_reserve_scratch(focr_ctx *handle, size_t bytes) {
  Ctx *ctx = reinterpret_cast<Ctx *>(handle);
  FOCR_REQUIRE(ctx, FOCR_E_ARG, "focr_ctx_reserve_scratch: null context");
  FOCR_HIP_CHECK(hipSetDevice(ctx->device));
  return ensure_scratch(ctx, bytes);
}

int focr_ctx_scratch_bytes(const focr_ctx *handle, size_t *bytes) {
  const Ctx *ctx = reinterpret_cast<const Ctx *>(handle);
  FOCR_REQUIRE(ctx && bytes, FOCR_E_ARG, "focr_ctx_scratch_bytes: null argument");
  *bytes = ctx->scratch_bytes;
  return FOCR_OK;
}

int focr_ctx_sync(focr_ctx *handle) {
  Ctx *ctx = reinterpret_cast<Ctx *>(handle);
  FOCR_REQUIRE(ctx, FOCR_E_ARG, "focr_ctx_sync: null context");
  FOCR_HIP_CHECK(hipStreamSynchronize(ctx->stream));
  return FOCR_OK;
}

int focr_malloc(focr_ctx *handle, size_t bytes, void **out) {
  Ctx *ctx = reinterpret_cast<Ctx *>(handle);
  FOCR_REQUIRE(ctx && out, FOCR_E_ARG, "focr_malloc: null argument");
  FOCR_HIP_CHECK(hipSetDevice(ctx->device));
  FOCR_HIP_CHECK(hipMalloc(out, bytes ? bytes : 1));
  return FOCR_OK;
}

int focr_free(focr_ctx *handle, void *dev) {
  Ctx *ctx = reinterpret_cast<Ctx *>(handle);
  FOCR_REQUIRE(ctx, FOCR_E_ARG, "focr_free: null context");
  if (dev) FOCR_HIP_CHECK(hipFree(dev));
  return FOCR_OK;
}

int focr_memcpy_h2d(focr_ctx *handle, void *dst, const void *src, size_t bytes) {
  Ctx *ctx = reinterpret_cast<Ctx *>(handle);
  FOCR_REQUIRE(ctx && (bytes == 0 || (dst && src)), FOCR_E_ARG, "focr_memcpy_h2d: null argument");
  FOCR_HIP_CHECK(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, ctx->stream));
  FOCR_HIP_CHECK(hipStreamSynchronize(ctx->stream));
  return FOCR_OK;
}

int focr_memcpy_d2h(focr_ctx *handle, void *dst, const void *src, size_t bytes) {
  Ctx *ctx = reinterpret_cast<Ctx *>(handle);
  FOCR_REQUIRE(ctx && (bytes == 0 || (dst && src)), FOCR_E_ARG, "focr_memcpy_d2h: null argument");
  FOCR_HIP_CHECK(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, ctx->stream));
  FOCR_HIP_CHECK(hipStreamSynchronize(ctx->stream));
  return FOCR_OK;
}

int focr_linear_upload(focr_ctx *handle, int bits, size_t n, size_t k, size_t group,
                       const void *codes, const float *scales, const int32_t *exc_cols,
                       const float *exc_vals, size_t n_exc, focr_linear **out) {
  Ctx *ctx = reinterpret_cast<Ctx *>(handle);
  FOCR_REQUIRE(ctx && out && codes, FOCR_E_ARG, "focr_linear_upload: null argument");
  FOCR_REQUIRE(bits == 8 || bits == 16 || bits == 32, FOCR_E_ARG, "focr_linear_upload: bits must be 8, 16 or 32");
  FOCR_REQUIRE(n > 0 && k > 0, FOCR_E_SHAPE, "focr_linear_upload: empty matrix");
  FOCR_REQUIRE(n <= (size_t(1) << 31) / 1 && k <= (size_t(1) << 24), FOCR_E_SHAPE,
               "focr_linear_upload: matrix too large");
  if (bits != 32) {
    FOCR_REQUIRE(group == 32 || group == 64 || group == 128, FOCR_E_SHAPE,
                 "focr_linear_upload: group must be 32, 64 or 128");
    FOCR_REQUIRE(scales, FOCR_E_ARG, "focr_linear_upload: null scales");
  } else {
    group = 32;
  }
  const size_t groups = (k + group - 1) / group;
  // from_parts' W8 rules (src/quant/linear.rs:330-351).
  if (bits == 8) {
    const int8_t *c8 = static_cast<const int8_t *>(codes);
    for (size_t i = 0; i < n * k; i++)
      FOCR_REQUIRE(c8[i] != -128, FOCR_E_VALUE, "W8 code -128 is outside [-127,127]");
    for (size_t i = 0; i < n * groups; i++) {
      const float s = scales[i];
      FOCR_REQUIRE(std::isfinite(s) && s >= 0.0f && std::isfinite(127.0f * s), FOCR_E_VALUE, "invalid W8 scale");
    }
    for (size_t row = 0; row < n; row++)
      for (size_t g = 0; g < groups; g++)
        if (scales[row * groups + g] == 0.0f)
          for (size_t i = g * group; i < std::min(k, (g + 1) * group); i++)
            FOCR_REQUIRE(c8[row * k + i] == 0, FOCR_E_VALUE, "nonzero code in zero-scale group");
  }
  // with_exceptions' rules (src/quant/linear.rs:366-390,437-452).
  if (n_exc) {
    FOCR_REQUIRE(bits != 32, FOCR_E_ARG, "exception columns need 8- or 16-bit codes");
    // The kernels find a column's exception through a 16-bit index per input.
    FOCR_REQUIRE(n_exc <= size_t(INT16_MAX), FOCR_E_UNSUPPORTED, "at most 32767 exception columns");
    FOCR_REQUIRE(exc_cols && exc_vals, FOCR_E_ARG, "focr_linear_upload: null exception arrays");
    for (size_t e = 0; e < n_exc; e++) {
      FOCR_REQUIRE(exc_cols[e] >= 0 && size_t(exc_cols[e]) < k, FOCR_E_VALUE, "exception column outside the inputs");
      FOCR_REQUIRE(e == 0 || exc_cols[e - 1] < exc_cols[e], FOCR_E_VALUE, "exception columns must be sorted and unique");
    }
    for (size_t i = 0; i < n * n_exc; i++)
      FOCR_REQUIRE(std::isfinite(exc_vals[i]), FOCR_E_VALUE, "nonfinite exception value");
    for (size_t e = 0; e < n_exc; e++)
      for (size_t row = 0; row < n; row++) {
        const size_t at = row * k + size_t(exc_cols[e]);
        const bool zero = bits == 8 ? static_cast<const int8_t *>(codes)[at] == 0
                                    : static_cast<const int16_t *>(codes)[at] == 0;
        FOCR_REQUIRE(zero, FOCR_E_VALUE, "nonzero code in an exception column");
      }
  }
  FOCR_HIP_CHECK(hipSetDevice(ctx->device));
  Linear *lin = new (std::nothrow) Linear();
  FOCR_REQUIRE(lin, FOCR_E_ARG, "focr_linear_upload: out of host memory");
  lin->bits = bits;
  lin->n = n;
  lin->k = k;
  lin->group = group;
  lin->groups = groups;
  lin->n_exc = n_exc;

  int rc = FOCR_OK;
  auto fail = [&](int code) {
    free_linear(lin);
    delete lin;
    return code;
  };
  const size_t cb = code_bytes(bits);
  size_t total = 0;
  {
    std::vector<uint8_t> raw(static_cast<const uint8_t *>(codes), static_cast<const uint8_t *>(codes) + n * k * cb);
    uint8_t *dev = nullptr;
    if ((rc = upload_vector(raw, &dev, &total)) != FOCR_OK) return fail(rc);
    lin->codes = dev;
  }
  if (bits != 32) {
    std::vector<float> s(scales, scales + n * groups);
    if ((rc = upload_vector(s, &lin->scales, &total)) != FOCR_OK) return fail(rc);
  }
  if (n_exc) {
    std::vector<int32_t> cols(exc_cols, exc_cols + n_exc);
    std::vector<float> vals(exc_vals, exc_vals + n * n_exc);
    std::vector<int16_t> index(k, -1);
    for (size_t e = 0; e < n_exc; e++) index[size_t(exc_cols[e])] = int16_t(e);
    if ((rc = upload_vector(cols, &lin->exc_cols, &total)) != FOCR_OK) return fail(rc);
    if ((rc = upload_vector(vals, &lin->exc_vals, &total)) != FOCR_OK) return fail(rc);
    if ((rc = upload_vector(index, &lin->exc_index, &total)) != FOCR_OK) return fail(rc);
  }
  // Decode GEMV tiles.
  {
    const size_t S = 16 / (2 * cb);
    const size_t nb = k / 32;
    lin->gemv_blocks = nb;
    lin->gemv_tiles = (n + kGemvChannels - 1) / kGemvChannels;
    lin->gemv_steps = std::max<size_t>(1, (nb + S - 1) / S);
    lin->gemv_sps = bits == 32 ? 0 : (S * 32) / group;
    std::vector<uint8_t> tiled;
    std::vector<float> tiled_scales;
    if (bits == 8)
      build_gemv_tiles(*lin, static_cast<const int8_t *>(codes), scales, tiled, tiled_scales);
    else if (bits == 16)
      build_gemv_tiles(*lin, static_cast<const int16_t *>(codes), scales, tiled, tiled_scales);
    else
      build_gemv_tiles(*lin, static_cast<const float *>(codes), scales, tiled, tiled_scales);
    uint8_t *dev = nullptr;
    if ((rc = upload_vector(tiled, &dev, &total)) != FOCR_OK) return fail(rc);
    lin->gemv_codes = dev;
    if ((rc = upload_vector(tiled_scales, &lin->gemv_scales, &total)) != FOCR_OK) return fail(rc);
  }
  // INT16-panel operands (fits_i16_panels, src/quant/linear.rs:29-31).
  if (bits == 8 && group == 64 && n % 32 == 0 && k % 64 == 0) {
    const int8_t *c8 = static_cast<const int8_t *>(codes);
    const size_t nblk = n / 16;
    std::vector<int8_t> b(groups * nblk * 1024);
    std::vector<int32_t> wsum(groups * n);
    std::vector<float> sw(groups * n);
    for (size_t g = 0; g < groups; g++)
      for (size_t blk = 0; blk < nblk; blk++)
        for (size_t lane = 0; lane < 64; lane++)
          for (size_t j = 0; j < 16; j++)
            b[((g * nblk + blk) * 64 + lane) * 16 + j] = c8[(blk * 16 + lane % 16) * k + g * 64 + 16 * (lane / 16) + j];
    for (size_t g = 0; g < groups; g++)
      for (size_t col = 0; col < n; col++) {
        int32_t s = 0;
        for (size_t j = 0; j < 64; j++) s += c8[col * k + g * 64 + j];
        wsum[g * n + col] = 128 * s;
        sw[g * n + col] = scales[col * groups + g];
      }
    if ((rc = upload_vector(b, &lin->i16_b, &total)) != FOCR_OK) return fail(rc);
    if ((rc = upload_vector(wsum, &lin->i16_wsum, &total)) != FOCR_OK) return fail(rc);
    if ((rc = upload_vector(sw, &lin->i16_sw, &total)) != FOCR_OK) return fail(rc);
  }
  // FP16 pairs of FP32 weights (FOCR_PROJ_F32_SPLIT's B operand).
  if (bits == 32 && (rc = prepare_pairs(ctx, lin, &total)) != FOCR_OK) return fail(rc);
  lin->device_bytes = total;
  *out = reinterpret_cast<focr_linear *>(lin);
  return FOCR_OK;
}

int focr_linear_free(focr_linear *handle) {
  Linear *lin = reinterpret_cast<Linear *>(handle);
  if (!lin) return FOCR_OK;
  free_linear(lin);
  delete lin;
  return FOCR_OK;
}

int focr_linear_info(const focr_linear *handle, int *bits, size_t *n, size_t *k, size_t *group,
                     size_t *n_exc, size_t *device_bytes) {
  const Linear *lin = reinterpret_cast<const Linear *>(handle);
  FOCR_REQUIRE(lin, FOCR_E_ARG, "focr_linear_info: null matrix");
  if (bits) *bits = lin->bits;
  if (n) *n = lin->n;
  if (k) *k = lin->k;
  if (group) *group = lin->group;
  if (n_exc) *n_exc = lin->n_exc;
  if (device_bytes) *device_bytes = lin->device_bytes;
  return FOCR_OK;
}

int focr_linear_dequantize(focr_ctx *handle, const focr_linear *lh, float *out) {
  Ctx *ctx = reinterpret_cast<Ctx *>(handle);
  const Linear *lin = reinterpret_cast<const Linear *>(lh);
  FOCR_REQUIRE(ctx && lin && out, FOCR_E_ARG, "focr_linear_dequantize: null argument");
  return launch_dequantize(ctx, lin, out);
}

int focr_linear_decode(focr_ctx *handle, const focr_linear *lh, const float *x, size_t rows, float *out) {
  Ctx *ctx = reinterpret_cast<Ctx *>(handle);
  const Linear *lin = reinterpret_cast<const Linear *>(lh);
  FOCR_REQUIRE(ctx && lin, FOCR_E_ARG, "focr_linear_decode: null argument");
  FOCR_REQUIRE(rows <= 8, FOCR_E_SHAPE, "focr_linear_decode: 1..=8 rows (decode and draft verification)");
  if (rows == 0) return FOCR_OK;
  FOCR_REQUIRE(x && out, FOCR_E_ARG, "focr_linear_decode: null buffer");
  return launch_gemv(ctx, lin, x, rows, nullptr, FOCR_EPI_STORE, out);
}

int focr_linear_decode_glu(focr_ctx *handle, const focr_linear *lh, const float *x, size_t rows, float *gated) {
  Ctx *ctx = reinterpret_cast<Ctx *>(handle);
  const Linear *lin = reinterpret_cast<const Linear *>(lh);
  FOCR_REQUIRE(ctx && lin, FOCR_E_ARG, "focr_linear_decode_glu: null argument");
  FOCR_REQUIRE(lin->n % 2 == 0, FOCR_E_SHAPE, "GLU needs interleaved gate/up rows");
  FOCR_REQUIRE(rows <= 8, FOCR_E_SHAPE, "focr_linear_decode_glu: 1..=8 rows");
  if (rows == 0) return FOCR_OK;
  FOCR_REQUIRE(x && gated, FOCR_E_ARG, "focr_linear_decode_glu: null buffer");
  return launch_gemv(ctx, lin, x, rows, nullptr, FOCR_EPI_GLU, gated);
}

int focr_linear_decode_ex(focr_ctx *handle, const focr_linear *lh, const float *x, size_t rows,
                          const float *row_scale, int rms_norm, int epilogue, float *out) {
  Ctx *ctx = reinterpret_cast<Ctx *>(handle);
  const Linear *lin = reinterpret_cast<const Linear *>(lh);
  FOCR_REQUIRE(ctx && lin, FOCR_E_ARG, "focr_linear_decode_ex: null argument");
  FOCR_REQUIRE(epilogue == FOCR_EPI_STORE || epilogue == FOCR_EPI_GLU || epilogue == FOCR_EPI_ADD, FOCR_E_ARG,
               "focr_linear_decode_ex: unknown epilogue");
  FOCR_REQUIRE(epilogue != FOCR_EPI_GLU || lin->n % 2 == 0, FOCR_E_SHAPE, "GLU needs interleaved gate/up rows");
  FOCR_REQUIRE(rows <= 8, FOCR_E_SHAPE, "focr_linear_decode_ex: 1..=8 rows (decode and draft verification)");
  FOCR_REQUIRE(rms_norm == 0 || rms_norm == 1, FOCR_E_ARG, "focr_linear_decode_ex: rms_norm is 0 or 1");
  FOCR_REQUIRE(!(rms_norm && row_scale), FOCR_E_ARG, "focr_linear_decode_ex: rms_norm and row_scale are exclusive");
  if (rows == 0) return FOCR_OK;
  FOCR_REQUIRE(x && out, FOCR_E_ARG, "focr_linear_decode_ex: null buffer");
  FOCR_HIP_CHECK(hipSetDevice(ctx->device));
  return launch_gemv(ctx, lin, x, rows, row_scale, epilogue, out, rms_norm != 0);
}

int focr_linear_prefill(focr_ctx *handle, const focr_linear *lh, const float *x, size_t rows,
                        const float *row_scale, int epilogue, int kernel, float *out) {
  Ctx *ctx = reinterpret_cast<Ctx *>(handle);
  const Linear *lin = reinterpret_cast<const Linear *>(lh);
  FOCR_REQUIRE(ctx && lin, FOCR_E_ARG, "focr_linear_prefill: null argument");
  FOCR_REQUIRE(epilogue == FOCR_EPI_STORE || epilogue == FOCR_EPI_GLU || epilogue == FOCR_EPI_ADD,
               FOCR_E_ARG, "focr_linear_prefill: unknown epilogue");
  FOCR_REQUIRE(epilogue != FOCR_EPI_GLU || lin->n % 2 == 0, FOCR_E_SHAPE, "GLU needs interleaved gate/up rows");
  if (rows == 0) return FOCR_OK;
  FOCR_REQUIRE(x && out, FOCR_E_ARG, "focr_linear_prefill: null buffer");
  FOCR_HIP_CHECK(hipSetDevice(ctx->device));
  switch (kernel) {
    case FOCR_PROJ_F32_MFMA:
      return launch_prefill_f32(ctx, lin, x, rows, row_scale, epilogue, out);
    case FOCR_PROJ_F32_CHAIN:
      return launch_prefill_chain(ctx, lin, x, rows, row_scale, epilogue, out);
    case FOCR_PROJ_F32_SPLIT:
      return launch_prefill_split(ctx, lin, x, rows, row_scale, epilogue, out);
    case FOCR_PROJ_I16:
      FOCR_REQUIRE(lin->i16_b, FOCR_E_UNSUPPORTED,
                   "the INT16 panels take 8-bit codes in groups of 64 with out % 32 == 0 and in % 64 == 0 "
                   "(fits_i16_panels); plan the FP32 panels for this matrix");
      return launch_prefill_i16(ctx, lin, x, rows, row_scale, epilogue, out);
    default:
      return set_error(FOCR_E_ARG, "focr_linear_prefill: unknown kernel");
  }
}

int focr_row_scales(focr_ctx *handle, const float *h, size_t rows, size_t width, float eps, float *out) {
  Ctx *ctx = reinterpret_cast<Ctx *>(handle);
  FOCR_REQUIRE(ctx, FOCR_E_ARG, "focr_row_scales: null context");
  FOCR_REQUIRE(width > 0, FOCR_E_SHAPE, "RMSNorm width must be positive");
  FOCR_REQUIRE(std::isfinite(eps) && eps > 0.0f, FOCR_E_ARG, "RMSNorm epsilon must be finite and positive");
  if (rows == 0) return FOCR_OK;
  FOCR_REQUIRE(h && out, FOCR_E_ARG, "focr_row_scales: null buffer");
  return launch_row_scales(ctx, h, rows, width, eps, out);
}

int focr_attention_prefill(focr_ctx *handle, const float *q, const float *prefix_k, const float *generated_k,
                           const float *v, size_t query_len, size_t prefix_len, size_t total_len,
                           size_t n_heads, size_t n_kv_heads, size_t head_dim, size_t query_offset,
                           size_t image_start, size_t image_end, const float *sinks, int softmax,
                           int exp_mode, float *out) {
  Ctx *ctx = reinterpret_cast<Ctx *>(handle);
  FOCR_REQUIRE(ctx, FOCR_E_ARG, "focr_attention_prefill: null context");
  // CompactKv::validate (src/kernels/attention/mod.rs:157-195).
  FOCR_REQUIRE(head_dim > 0 && n_heads > 0 && n_kv_heads > 0, FOCR_E_SHAPE, "attention head dimensions must be positive");
  FOCR_REQUIRE(head_dim == 64, FOCR_E_UNSUPPORTED, "the hip attention tiles take head_dim 64");
  FOCR_REQUIRE(n_heads % n_kv_heads == 0, FOCR_E_SHAPE, "attention GQA grouping");
  FOCR_REQUIRE(prefix_len <= total_len, FOCR_E_SHAPE, "attention prefix length");
  FOCR_REQUIRE(image_start <= image_end && image_end <= prefix_len, FOCR_E_SHAPE, "attention image must be inside the prefix");
  FOCR_REQUIRE(query_offset + query_len <= total_len, FOCR_E_SHAPE, "attention query interval");
  FOCR_REQUIRE(softmax == FOCR_SOFTMAX_ONLINE || softmax == FOCR_SOFTMAX_STATIC, FOCR_E_ARG, "unknown softmax");
  FOCR_REQUIRE(exp_mode == FOCR_EXP_FAST || exp_mode == FOCR_EXP_EXACT, FOCR_E_ARG, "unknown exp mode");
  FOCR_REQUIRE(softmax != FOCR_SOFTMAX_STATIC || prefix_len == total_len, FOCR_E_SHAPE,
               "the static-shift tiles take pure prefixes");
  if (query_len == 0) return FOCR_OK;
  FOCR_REQUIRE(q && prefix_k && v && sinks && out, FOCR_E_ARG, "focr_attention_prefill: null buffer");
  FOCR_REQUIRE(prefix_len == total_len || generated_k, FOCR_E_ARG, "generated keys missing");
  FOCR_HIP_CHECK(hipSetDevice(ctx->device));
  return launch_attention(ctx, q, prefix_k, generated_k, v, query_len, prefix_len, total_len, n_heads,
                          n_kv_heads, query_offset, image_start, image_end, sinks, softmax, exp_mode, out);
}

int focr_attention_prefill_split(focr_ctx *handle, const float *q, const float *prefix_k, const float *generated_k,
                                 const float *v, size_t query_len, size_t prefix_len, size_t total_len,
                                 size_t n_heads, size_t n_kv_heads, size_t head_dim, size_t query_offset,
                                 size_t image_start, size_t image_end, const float *sinks, int softmax,
                                 int exp_mode, float *out) {
  Ctx *ctx = reinterpret_cast<Ctx *>(handle);
  FOCR_REQUIRE(ctx, FOCR_E_ARG, "focr_attention_prefill_split: null context");
  FOCR_REQUIRE(head_dim > 0 && n_heads > 0 && n_kv_heads > 0, FOCR_E_SHAPE, "attention head dimensions must be positive");
  FOCR_REQUIRE(head_dim == 64, FOCR_E_UNSUPPORTED, "the hip attention tiles take head_dim 64");
  FOCR_REQUIRE(n_heads % n_kv_heads == 0, FOCR_E_SHAPE, "attention GQA grouping");
  FOCR_REQUIRE(prefix_len <= total_len, FOCR_E_SHAPE, "attention prefix length");
  FOCR_REQUIRE(image_start <= image_end && image_end <= prefix_len, FOCR_E_SHAPE, "attention image must be inside the prefix");
  FOCR_REQUIRE(query_offset + query_len <= total_len, FOCR_E_SHAPE, "attention query interval");
  FOCR_REQUIRE(softmax == FOCR_SOFTMAX_ONLINE || softmax == FOCR_SOFTMAX_STATIC, FOCR_E_ARG, "unknown softmax");
  FOCR_REQUIRE(exp_mode == FOCR_EXP_FAST || exp_mode == FOCR_EXP_EXACT, FOCR_E_ARG, "unknown exp mode");
  FOCR_REQUIRE(query_offset == 0 && query_len == prefix_len && prefix_len == total_len, FOCR_E_UNSUPPORTED,
               "the split-product attention takes pure prefills; focr_attention_prefill takes the rest");
  if (query_len == 0) return FOCR_OK;
  FOCR_REQUIRE(q && prefix_k && v && sinks && out, FOCR_E_ARG, "focr_attention_prefill_split: null buffer");
  FOCR_HIP_CHECK(hipSetDevice(ctx->device));
  return launch_attention_split(ctx, q, prefix_k, v, query_len, n_heads, n_kv_heads, image_start, image_end, sinks,
                                softmax, exp_mode, out);
}

int focr_attention_prefill_bf16(focr_ctx *handle, const float *q, const float *k, const float *v, size_t query_len,
                                size_t n_heads, size_t n_kv_heads, size_t head_dim, size_t image_start,
                                size_t image_end, const float *sinks, int softmax, int exp_mode, float *out) {
  Ctx *ctx = reinterpret_cast<Ctx *>(handle);
  FOCR_REQUIRE(ctx, FOCR_E_ARG, "focr_attention_prefill_bf16: null context");
  // CompactKv::validate (src/kernels/attention/mod.rs:157-195) for a pure prefill.
  FOCR_REQUIRE(head_dim > 0 && n_heads > 0 && n_kv_heads > 0, FOCR_E_SHAPE, "attention head dimensions must be positive");
  FOCR_REQUIRE(n_heads % n_kv_heads == 0, FOCR_E_SHAPE, "attention GQA grouping");
  FOCR_REQUIRE(image_start <= image_end && image_end <= query_len, FOCR_E_SHAPE, "attention image must be inside the prefix");
  FOCR_REQUIRE(softmax == FOCR_SOFTMAX_ONLINE || softmax == FOCR_SOFTMAX_STATIC, FOCR_E_ARG, "unknown softmax");
  FOCR_REQUIRE(exp_mode == FOCR_EXP_FAST || exp_mode == FOCR_EXP_EXACT, FOCR_E_ARG, "unknown exp mode");
  // attention_prefill_bf16 (mod.rs:320-352) runs only these shapes and
  // otherwise returns false: here FOCR_E_UNSUPPORTED, nothing written.
  FOCR_REQUIRE(query_len >= 4 && head_dim == 64, FOCR_E_UNSUPPORTED,
               "the BF16 attention takes pure prefills of at least 4 queries with head_dim 64");
  FOCR_REQUIRE(q && k && v && sinks && out, FOCR_E_ARG, "focr_attention_prefill_bf16: null buffer");
  FOCR_HIP_CHECK(hipSetDevice(ctx->device));
  return launch_attention_bf16(ctx, q, k, v, query_len, n_heads, n_kv_heads, image_start, image_end, sinks, softmax,
                               out);
}

int focr_qkv_rows(focr_ctx *handle, const float *qkv, size_t rows, const float *rope, size_t n_heads,
                  size_t n_kv_heads, size_t head_dim, size_t prefix_rows, float *q, float *prefix_k,
                  float *generated_k, float *v) {
  Ctx *ctx = reinterpret_cast<Ctx *>(handle);
  FOCR_REQUIRE(ctx, FOCR_E_ARG, "focr_qkv_rows: null context");
  FOCR_REQUIRE(n_heads > 0 && n_kv_heads > 0 && n_heads % n_kv_heads == 0, FOCR_E_SHAPE, "qkv rows: GQA grouping");
  FOCR_REQUIRE(head_dim == 64, FOCR_E_UNSUPPORTED, "the hip QKV row kernel takes head_dim 64");
  FOCR_REQUIRE(prefix_rows <= rows, FOCR_E_SHAPE, "qkv rows: more prefix rows than rows");
  if (rows == 0) return FOCR_OK;
  FOCR_REQUIRE(qkv && rope && q && v, FOCR_E_ARG, "focr_qkv_rows: null buffer");
  FOCR_REQUIRE(prefix_rows == 0 || prefix_k, FOCR_E_ARG, "focr_qkv_rows: prefix keys missing");
  FOCR_REQUIRE(prefix_rows == rows || generated_k, FOCR_E_ARG, "focr_qkv_rows: generated keys missing");
  FOCR_HIP_CHECK(hipSetDevice(ctx->device));
  return launch_qkv_rows(ctx, qkv, rows, rope, n_heads, n_kv_heads, prefix_rows, q, prefix_k, generated_k, v);
}

int focr_attention_decode(focr_ctx *handle, const float *q, const float *prefix_k, const float *generated_k,
                          const float *v, size_t query_len, size_t prefix_len, size_t total_len, size_t n_heads,
                          size_t n_kv_heads, size_t head_dim, size_t query_offset, size_t image_start,
                          size_t image_end, const float *sinks, float *out) {
  Ctx *ctx = reinterpret_cast<Ctx *>(handle);
  FOCR_REQUIRE(ctx, FOCR_E_ARG, "focr_attention_decode: null context");
  // CompactKv::validate (src/kernels/attention/mod.rs:157-195).
  FOCR_REQUIRE(head_dim > 0 && n_heads > 0 && n_kv_heads > 0, FOCR_E_SHAPE, "attention head dimensions must be positive");
  FOCR_REQUIRE(head_dim == 64, FOCR_E_UNSUPPORTED, "the hip decode attention takes head_dim 64");
  FOCR_REQUIRE(n_heads % n_kv_heads == 0, FOCR_E_SHAPE, "attention GQA grouping");
  FOCR_REQUIRE(prefix_len <= total_len, FOCR_E_SHAPE, "attention prefix length");
  FOCR_REQUIRE(image_start <= image_end && image_end <= prefix_len, FOCR_E_SHAPE, "attention image must be inside the prefix");
  FOCR_REQUIRE(query_offset + query_len <= total_len, FOCR_E_SHAPE, "attention query interval");
  FOCR_REQUIRE(query_len <= 8, FOCR_E_SHAPE, "decode attention takes 1..=8 query rows");
  if (query_len == 0) return FOCR_OK;
  FOCR_REQUIRE(q && v && sinks && out, FOCR_E_ARG, "focr_attention_decode: null buffer");
  FOCR_REQUIRE(prefix_len == 0 || prefix_k, FOCR_E_ARG, "prefix keys missing");
  FOCR_REQUIRE(prefix_len == total_len || generated_k, FOCR_E_ARG, "generated keys missing");
  FOCR_HIP_CHECK(hipSetDevice(ctx->device));
  return launch_attention_decode(ctx, q, prefix_k, generated_k, v, query_len, prefix_len, total_len, n_heads,
                                 n_kv_heads, query_offset, image_start, image_end, sinks, out);
}

int focr_attention_decode_row(focr_ctx *handle, const float *qkv, const float *rope, const float *prefix_k,
                              float *generated_k, float *v, size_t prefix_len, size_t total_len, size_t n_heads,
                              size_t n_kv_heads, size_t head_dim, size_t image_start, size_t image_end,
                              const float *sinks, float *q, float *out) {
  Ctx *ctx = reinterpret_cast<Ctx *>(handle);
  FOCR_REQUIRE(ctx, FOCR_E_ARG, "focr_attention_decode_row: null context");
  FOCR_REQUIRE(head_dim > 0 && n_heads > 0 && n_kv_heads > 0, FOCR_E_SHAPE, "attention head dimensions must be positive");
  FOCR_REQUIRE(head_dim == 64, FOCR_E_UNSUPPORTED, "the hip decode attention takes head_dim 64");
  FOCR_REQUIRE(n_heads % n_kv_heads == 0, FOCR_E_SHAPE, "attention GQA grouping");
  FOCR_REQUIRE(prefix_len < total_len, FOCR_E_SHAPE, "the decode row is a generated row: prefix_len < total_len");
  FOCR_REQUIRE(image_start <= image_end && image_end <= prefix_len, FOCR_E_SHAPE, "attention image must be inside the prefix");
  FOCR_REQUIRE(qkv && rope && generated_k && v && sinks && out, FOCR_E_ARG, "focr_attention_decode_row: null buffer");
  FOCR_REQUIRE(prefix_len == 0 || prefix_k, FOCR_E_ARG, "prefix keys missing");
  FOCR_HIP_CHECK(hipSetDevice(ctx->device));
  return launch_attention_decode_row(ctx, qkv, rope, prefix_k, generated_k, v, prefix_len, total_len, n_heads,
                                     n_kv_heads, image_start, image_end, sinks, q, out);
}

int focr_argmax(focr_ctx *handle, const float *logits, size_t rows, size_t vocab, uint32_t *tokens) {
  Ctx *ctx = reinterpret_cast<Ctx *>(handle);
  FOCR_REQUIRE(ctx, FOCR_E_ARG, "focr_argmax: null context");
  FOCR_REQUIRE(vocab > 0 && vocab < (size_t(1) << 31), FOCR_E_NONFINITE, "nonfinite or empty logits");
  if (rows == 0) return FOCR_OK;
  FOCR_REQUIRE(logits && tokens, FOCR_E_ARG, "focr_argmax: null buffer");
  FOCR_HIP_CHECK(hipSetDevice(ctx->device));
  if (ctx->argmax_rows < rows) {
    if (ctx->argmax_dev) {
      FOCR_HIP_CHECK(hipStreamSynchronize(ctx->stream));
      FOCR_HIP_CHECK(hipFree(ctx->argmax_dev));
      ctx->argmax_dev = nullptr;
    }
    FOCR_HIP_CHECK(hipMalloc(&ctx->argmax_dev, rows * 2 * sizeof(uint32_t)));
    ctx->argmax_rows = rows;
  }
  int rc = launch_argmax(ctx, logits, rows, vocab, ctx->argmax_dev);
  if (rc != FOCR_OK) return rc;
  std::vector<uint32_t> result(rows * 2);
  FOCR_HIP_CHECK(hipMemcpyAsync(result.data(), ctx->argmax_dev, rows * 2 * sizeof(uint32_t), hipMemcpyDeviceToHost, ctx->stream));
  FOCR_HIP_CHECK(hipStreamSynchronize(ctx->stream));
  for (size_t r = 0; r < rows; r++) {
    FOCR_REQUIRE(result[2 * r + 1] == 0, FOCR_E_NONFINITE, "nonfinite or empty logits");
    tokens[r] = result[2 * r];
  }
  return FOCR_OK;
}

}  // extern "C"
