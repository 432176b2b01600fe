// One block type's instances of the matvec and dequant kernels. The build compiles this file once per
// type, with -DSTRATA_KIND=<GGUF type id>, so the types compile in parallel.
#include "direct_impl.h"

#ifndef STRATA_KIND
#error "STRATA_KIND must name a GGUF type id"
#endif

#define STRATA_CAT2(a, b) a##b
#define STRATA_CAT(a, b) STRATA_CAT2(a, b)

namespace strata_mv {

int STRATA_CAT(matvec_launch_, STRATA_KIND)(MatvecParams& p, int x_dtype, int out_dtype, bool glu, int grid_y,
                                            int grid_z, hipStream_t s) {
  return launch_matvec_any<STRATA_KIND>(p, x_dtype, out_dtype, glu, grid_y, grid_z, s);
}

int STRATA_CAT(dequant_launch_, STRATA_KIND)(const uint8_t* blocks, int64_t runs_total, int runs_per_row,
                                             int row_bytes, void* out, int out_dtype, hipStream_t s) {
  return launch_dequant_kind<STRATA_KIND>(blocks, runs_total, runs_per_row, row_bytes, out, out_dtype, s);
}

}  // namespace strata_mv
