// Decode GEMV instantiations for f32 weights (kernel: gemv_kernel.hpp).
#include "gemv_kernel.hpp"

namespace focr {
namespace gemv {

int launch_f32(Ctx *ctx, const Linear *lin, const float *x, size_t rows, float *out, bool glu) {
  return launch_rows<float, 0>(ctx, lin, x, rows, out, glu);
}

}  // namespace gemv
}  // namespace focr
