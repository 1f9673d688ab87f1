// Decode GEMV instantiations for i8 weights (kernel: gemv_kernel.hpp).
#include "gemv_kernel.hpp"

namespace focr {
namespace gemv {

int launch_i8(Ctx *ctx, const Linear *lin, const float *x, const float *rs, size_t rows, float *out, int epi) {
  switch (lin->group) {
    case 32: return launch_rows<int8_t, 8>(ctx, lin, x, rs, rows, out, epi);
    case 64: return launch_rows<int8_t, 4>(ctx, lin, x, rs, rows, out, epi);
    default: return launch_rows<int8_t, 2>(ctx, lin, x, rs, rows, out, epi);
  }
}

}  // namespace gemv
}  // namespace focr
