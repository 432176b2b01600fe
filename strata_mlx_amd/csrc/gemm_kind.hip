// One block type's instances of the prompt kernels; compiled once per type with -DSTRATA_KIND=<GGUF type id>.
#include "gemm_impl.h"
#include "prompt_impl.h"
#include "prompt_wide.h"

#ifndef STRATA_KIND
#error "STRATA_KIND must name a GGUF type id"
#endif

#define STRATA_CAT2(a, b) a##b
#define STRATA_CAT(a, b) STRATA_CAT2(a, b)

namespace strata_gemm {

int STRATA_CAT(gemm_launch_, STRATA_KIND)(GemmParams& p, int a_dtype, hipStream_t s) {
  // IQ3_S / IQ3_XXS / Q2_0 rows of whole 256-weight steps with float16 activations: the register-decode kernel,
  // whose row offsets within a matrix are 32-bit (larger matrices take the other kernel)
  if constexpr (strata_mv::FastTraits<STRATA_KIND>::supported) {
    if (a_dtype == DT_F16 && strata_prompt::prompt_takes(STRATA_KIND, p.cols) && p.mat_bytes < (int64_t(1) << 32)) {
      strata_prompt::PromptParams q = {};
      q.blocks[0] = p.blocks;
      q.a = reinterpret_cast<const f16*>(p.a);
      q.a_max = p.a_max;
      q.tile_expert = p.tile_expert;
      q.out = p.c;
      q.experts = p.experts;
      q.mat_bytes = p.mat_bytes;
      q.rows = p.rows;
      q.cols = p.cols;
      q.row_bytes = p.row_bytes;
      q.n_tiles = p.n_tiles;
      return strata_prompt::launch_prompt<STRATA_KIND, strata_prompt::PM_C32, float>(q, s);
    }
  }
  return launch_gemm_kind<STRATA_KIND>(p, a_dtype, s);
}

}  // namespace strata_gemm

namespace strata_prompt {

int STRATA_CAT(prompt_launch_, STRATA_KIND)(PromptParams& p, int mode, int out_dtype, hipStream_t s) {
  if constexpr (strata_mv::FastTraits<STRATA_KIND>::supported) {
    if (mode == PM_GLU) {
      if (out_dtype == DT_F16) return launch_prompt_split<STRATA_KIND, PM_GLU, f16>(p, s);
      if (out_dtype == DT_BF16) return launch_prompt_split<STRATA_KIND, PM_GLU, bf16_t>(p, s);
      return STRATA_ERR_DTYPE;
    }
    if (mode == PM_SCATTER) {
      if (out_dtype == DT_F16) return launch_prompt_split<STRATA_KIND, PM_SCATTER, f16>(p, s);
      if (out_dtype == DT_BF16) return launch_prompt_split<STRATA_KIND, PM_SCATTER, bf16_t>(p, s);
      return STRATA_ERR_DTYPE;
    }
    return STRATA_ERR_ARG;
  } else {
    (void)p;
    (void)mode;
    (void)out_dtype;
    (void)s;
    return STRATA_ERR_KIND;
  }
}

}  // namespace strata_prompt
