// Decode GEMV dispatch (kernel: gemv_kernel.hpp; one instantiation file per
// code type: gemv_i8.hip, gemv_i16.hip, gemv_f32.hip).
#include "gemv_kernel.hpp"

namespace focr {

// Largest row count whose x fits the 64 KB of LDS a workgroup may take
// (x is staged in LDS, padded to whole steps).
static size_t rows_per_launch(const Linear *lin) {
  const size_t scales = gemv::scale_lds_bytes(lin);
  const size_t fit = scales >= gemv::kLdsBudget ? 0 : (gemv::kLdsBudget - scales) / gemv::x_row_bytes(lin);
  return fit < 8 ? fit : 8;
}

int launch_gemv(Ctx *ctx, const Linear *lin, const float *x, size_t rows, const float *row_scale, int epilogue,
                float *out, bool rms_norm) {
  FOCR_HIP_CHECK(hipSetDevice(ctx->device));
  const size_t chunk = rows_per_launch(lin);
  FOCR_REQUIRE(chunk >= 1, FOCR_E_SHAPE, "GEMV: in_dim too large for one row of x in LDS");
  const size_t width = epilogue == FOCR_EPI_GLU ? lin->n / 2 : lin->n;
  // Rows are independent (each output row is its single-row dot, bitwise), so
  // a call whose inputs exceed the LDS budget runs as several launches.
  for (size_t r0 = 0; r0 < rows; r0 += chunk) {
    const size_t m = rows - r0 < chunk ? rows - r0 : chunk;
    const float *xr = x + r0 * lin->k;
    const float *rs = row_scale ? row_scale + r0 : nullptr;
    if (rms_norm && lin->k == static_cast<size_t>(gemv::kRmsWidth)) {
      rs = kRmsInKernel;
    } else if (rms_norm) {
      // Other widths: the row scales first, into the context's small buffer.
      int rc = launch_row_scales(ctx, xr, m, lin->k, 1.1920929e-7f, ctx->rms_dev);
      if (rc != FOCR_OK) return rc;
      rs = ctx->rms_dev;
    }
    float *orow = out + r0 * width;
    int rc;
    if (lin->bits == 8)
      rc = gemv::launch_i8(ctx, lin, xr, rs, m, orow, epilogue);
    else if (lin->bits == 16)
      rc = gemv::launch_i16(ctx, lin, xr, rs, m, orow, epilogue);
    else
      rc = gemv::launch_f32(ctx, lin, xr, rs, m, orow, epilogue);
    if (rc != FOCR_OK) return rc;
  }
  return FOCR_OK;
}

}  // namespace focr
