// One block type's instances of the prompt kernel; compiled once per type with -DSTRATA_KIND=<GGUF type id>.
#include "gemm_direct.h"

#ifndef STRATA_KIND
#error "STRATA_KIND must name a GGUF type id"
#endif

#define STRATA_CAT2(a, b) a##b
#define STRATA_CAT(a, b) STRATA_CAT2(a, b)

namespace strata_gemm {

int STRATA_CAT(gemm_launch_, STRATA_KIND)(GemmParams& p, int a_dtype, hipStream_t s) {
  // IQ3_S / IQ3_XXS / Q2_0 rows of whole 256-weight blocks with 16-bit activations: the direct kernel
  if constexpr (strata_mv::FastTraits<STRATA_KIND>::supported) {
    if ((a_dtype == DT_F16 || a_dtype == DT_BF16) && p.cols % kDStep == 0 && p.n_tiles <= 65535)
      return launch_direct_gemm<STRATA_KIND>(p, a_dtype, s);
  }
  return launch_gemm_kind<STRATA_KIND>(p, a_dtype, s);
}

}  // namespace strata_gemm
