// One part of the GEMM kernels for one channel capacity: built once per
// (RNSMX_RCAP, RNSMX_PART) pair so the library compiles in parallel.  The
// parts are listed beside gemm_part_of in rnsmx_gemm.hpp.
#include "rnsmx_gemm.hpp"

#if !defined(RNSMX_RCAP) || !defined(RNSMX_PART)
#error "build with -DRNSMX_RCAP=<3|4|6|10> -DRNSMX_PART=<0..5>"
#endif

#define RNSMX_PASTE_PART(R, P) RNSMX_GEMM_PART_NAME(R, P)

namespace rnsmx {
bool RNSMX_PASTE_PART(RNSMX_RCAP, RNSMX_PART)(const GemmArgs &g, bool araw, const GemmChoice &c,
                                              hipStream_t st) {
  return launch_gemm_part<RNSMX_RCAP, RNSMX_PART>(g, araw, c, st);
}
}  // namespace rnsmx
