// Decode GEMV instantiations for f32 weights (kernel: gemv_kernel.hpp).
#include "gemv_kernel.hpp"

namespace focr {
namespace gemv {

int launch_f32(Ctx *ctx, const Linear *lin, const float *x, const float *rs, size_t rows, float *out, int epi) {
  return launch_rows<float, 0>(ctx, lin, x, rs, rows, out, epi);
}

}  // namespace gemv
}  // namespace focr
