// One block type's instances of the prompt kernel; compiled once per type with -DSTRATA_KIND=<GGUF type id>.
#include "gemm_impl.h"

#ifndef STRATA_KIND
#error "STRATA_KIND must name a GGUF type id"
#endif

#define STRATA_CAT2(a, b) a##b
#define STRATA_CAT(a, b) STRATA_CAT2(a, b)

namespace strata_gemm {

int STRATA_CAT(gemm_launch_, STRATA_KIND)(GemmParams& p, int a_dtype, hipStream_t s) {
  return launch_gemm_kind<STRATA_KIND>(p, a_dtype, s);
}

}  // namespace strata_gemm
