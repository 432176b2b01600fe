// C-ABI entry point of the prompt kernel (declared in include/strata_gfx950.h); kernels in gemm_impl.h.
#include "gemm_impl.h"

namespace strata_gemm {
#define STRATA_DECLARE(K) int gemm_launch_##K(GemmParams&, int, hipStream_t);
STRATA_DECLARE(2)
STRATA_DECLARE(6)
STRATA_DECLARE(8)
STRATA_DECLARE(11)
STRATA_DECLARE(12)
STRATA_DECLARE(14)
STRATA_DECLARE(18)
STRATA_DECLARE(20)
STRATA_DECLARE(21)
STRATA_DECLARE(13)
STRATA_DECLARE(23)
STRATA_DECLARE(42)
#undef STRATA_DECLARE
}  // namespace strata_gemm

using namespace strata_gemm;

extern "C" int strata_grouped_matmul(int kind, const void* blocks, int64_t experts, int64_t rows, int64_t cols,
                                     const void* a, int a_dtype, const uint32_t* a_max, const uint32_t* tile_expert,
                                     int64_t n_tiles, int64_t tile, float* c, void* stream) {
  int per = 0, bb = 0;
  if (strata_kind_info(kind, &per, &bb)) return STRATA_ERR_KIND;
  if (rows < 0 || cols <= 0 || cols % per || cols % kKStep || rows > (1 << 24) || cols > (1 << 20))
    return STRATA_ERR_SHAPE;
  if (a_dtype != DT_F32 && a_dtype != DT_F16) return STRATA_ERR_DTYPE;
  if (a_max && a_dtype != DT_F16) return STRATA_ERR_ARG;
  if (tile != 16 || n_tiles < 0 || experts < 0) return STRATA_ERR_ARG;
  if (n_tiles == 0 || rows == 0) return STRATA_OK;
  if (!blocks || !a || !tile_expert || !c) return STRATA_ERR_ARG;
  GemmParams p = {};
  p.blocks = (const uint8_t*)blocks;
  p.a = a;
  p.a_max = a_max;
  p.tile_expert = tile_expert;
  p.c = c;
  p.experts = experts;
  p.rows = (int)rows;
  p.cols = (int)cols;
  p.row_bytes = (int)(cols / per * bb);
  p.mat_bytes = rows * (int64_t)p.row_bytes;
  p.n_tiles = (int)n_tiles;
  hipStream_t s = (hipStream_t)stream;
  switch (kind) {
#define STRATA_CASE(K) \
  case K: return gemm_launch_##K(p, a_dtype, s);
    STRATA_CASE(2)
    STRATA_CASE(6)
    STRATA_CASE(8)
    STRATA_CASE(11)
    STRATA_CASE(12)
    STRATA_CASE(14)
    STRATA_CASE(18)
    STRATA_CASE(20)
    STRATA_CASE(21)
    STRATA_CASE(13)
    STRATA_CASE(23)
    STRATA_CASE(42)
#undef STRATA_CASE
    default: return STRATA_ERR_KIND;
  }
}
