// GEMM kernels for moduli sets of up to 10 channels (one translation unit
// per channel capacity so the library builds in parallel).
#include "rnsmx_gemm.hpp"

namespace rnsmx {
bool launch_gemm_r10(const GemmArgs &g, bool araw, const GemmChoice &c, hipStream_t st) {
  return launch_gemm_rcap<10>(g, araw, c, st);
}
}  // namespace rnsmx
