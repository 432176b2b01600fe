// C-ABI entry points of the dequant and matvec family (declared in include/strata_gfx950.h).
// Arguments are checked here; the kernels live in matvec_impl.h, one object per block type.
#include "matvec_impl.h"

namespace strata_mv {
#define STRATA_DECLARE(K)                                                                                    \
  int matvec_launch_##K(MatvecParams&, int, int, bool, int, int, hipStream_t);                              \
  int dequant_launch_##K(const uint8_t*, int64_t, int, int, void*, int, hipStream_t);
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
}  // namespace strata_mv

using namespace strata_mv;

namespace {

int launch_by_kind(int kind, MatvecParams& p, int x_dtype, int out_dtype, bool glu, int gy, int gz, hipStream_t s) {
  switch (kind) {
#define STRATA_CASE(K) \
  case K: return matvec_launch_##K(p, x_dtype, out_dtype, glu, gy, gz, s);
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

int dequant_by_kind(int kind, const uint8_t* b, int64_t runs, int per_row, int row_bytes, void* out, int dt,
                    hipStream_t s) {
  switch (kind) {
#define STRATA_CASE(K) \
  case K: return dequant_launch_##K(b, runs, per_row, row_bytes, out, dt, s);
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

int block_shape(int kind, int64_t rows, int64_t cols, int* row_bytes) {
  int per = 0, bb = 0;
  if (strata_kind_info(kind, &per, &bb)) return STRATA_ERR_KIND;
  if (rows < 0 || cols <= 0 || cols % per || cols % 32) return STRATA_ERR_SHAPE;
  if (rows > (1 << 30) || cols > (1 << 20)) return STRATA_ERR_SHAPE;
  *row_bytes = (int)(cols / per * bb);
  return STRATA_OK;
}

bool valid_dtype(int dt) { return dt == DT_F32 || dt == DT_F16 || dt == DT_BF16; }

template <typename XT>
__global__ void swiglu_kernel(const XT* g, const XT* u, XT* h, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) h[i] = from_f32<XT>(swiglu_rounded<XT>(g[i], u[i]));
}

// h = silu(g) * u over n elements, rounded as mlx-lm rounds it
int launch_swiglu(const void* g, const void* u, void* h, int64_t n, int dtype, hipStream_t s) {
  const int64_t blocks = (n + 255) / 256;
  if (blocks > INT32_MAX) return STRATA_ERR_SHAPE;
  if (dtype == DT_F16)
    hipLaunchKernelGGL(swiglu_kernel<f16>, dim3((int)blocks), dim3(256), 0, s, (const f16*)g, (const f16*)u, (f16*)h, n);
  else if (dtype == DT_BF16)
    hipLaunchKernelGGL(swiglu_kernel<bf16_t>, dim3((int)blocks), dim3(256), 0, s, (const bf16_t*)g, (const bf16_t*)u,
                       (bf16_t*)h, n);
  else
    hipLaunchKernelGGL(swiglu_kernel<float>, dim3((int)blocks), dim3(256), 0, s, (const float*)g, (const float*)u,
                       (float*)h, n);
  STRATA_CHECK_LAUNCH();
  return STRATA_OK;
}

int expert_common(int kind, const void* a, const void* b, int64_t experts, int64_t rows, int64_t cols,
                  const uint32_t* idx, int64_t pairs, const void* x, const void* up, int dtype, int64_t share,
                  void* out_a, void* out_b, bool glu, void* stream, void* out_h = nullptr) {
  MatvecParams p = {};
  int rc = block_shape(kind, rows, cols, &p.row_bytes);
  if (rc) return rc;
  if (!valid_dtype(dtype)) return STRATA_ERR_DTYPE;
  if (pairs < 0 || experts < 0 || experts > INT32_MAX) return STRATA_ERR_ARG;
  if (pairs == 0 || rows == 0) return STRATA_OK;
  if (experts == 0 || !a || !idx || !x || !out_a || (b && !out_b) || (glu && !up)) return STRATA_ERR_ARG;
  if (share < 1 || pairs % share) return STRATA_ERR_ARG;
  if (pairs > 65535 || cols / 32 > 256) return STRATA_ERR_SHAPE;
  p.blocks[0] = (const uint8_t*)a;
  p.blocks[1] = (const uint8_t*)b;
  p.out[0] = out_a;
  p.out[1] = out_b;
  p.idx = idx;
  p.x = x;
  p.up = up;
  p.mat_bytes = rows * (int64_t)p.row_bytes;
  p.experts = experts;
  p.src_rows = (int)rows;
  p.rows = (int)rows;
  p.cols = (int)cols;
  p.pairs = (int)pairs;
  p.share = (int)share;
  p.mode = MODE_EXPERT;
  if (out_h != nullptr) {  // gate and up with silu(gate) * up: one launch where the float16 kernels take it
    p.glu_out = out_h;
    rc = launch_by_kind(kind, p, dtype, dtype, false, (int)pairs, 2, (hipStream_t)stream);
    if (rc != STRATA_ERR_SHAPE) return rc;
    p.glu_out = nullptr;
    rc = launch_by_kind(kind, p, dtype, dtype, false, (int)pairs, 2, (hipStream_t)stream);
    if (rc) return rc;
    return launch_swiglu(out_a, out_b, out_h, pairs * rows, dtype, (hipStream_t)stream);
  }
  return launch_by_kind(kind, p, dtype, dtype, glu, (int)pairs, b ? 2 : 1, (hipStream_t)stream);
}

}  // namespace

// The routed gate/up launch at one token with a shared expert's gate and up in it, the pairs' experts given (idx)
// or chosen in the launch from the router's logits (logits not null: idx is then where the choice goes).
static int gate_up_shared(int kind, const void* gate_blocks, const void* up_blocks, int64_t experts, int64_t rows,
                          int64_t cols, const uint32_t* idx, int64_t pairs, const void* x, int x_dtype,
                          void* out_gate, void* out_up, void* out_h, int shared_kind, const void* shared_gate,
                          const void* shared_up, int64_t shared_rows, void* shared_h, void* shared_g, void* shared_u,
                          const float* logits, int64_t logit_rows, int64_t route_experts, uint32_t* idx_out,
                          float* w_out, void* extra_out, void* stream) {
  MatvecParams p = {};
  int rc = block_shape(kind, rows, cols, &p.row_bytes);
  if (rc) return rc;
  int s_row_bytes = 0;
  rc = block_shape(shared_kind, shared_rows, cols, &s_row_bytes);
  if (rc) return rc;
  if (x_dtype != DT_F16) return STRATA_ERR_DTYPE;
  if (pairs < 1 || experts < 1 || experts > INT32_MAX || shared_rows < 1) return STRATA_ERR_ARG;
  if (rows == 0) return STRATA_ERR_SHAPE;  // no routed launch to carry the shared expert: the two calls apart
  if (!gate_blocks || !up_blocks || !idx || !x || !out_h || !shared_gate || !shared_up || !shared_h)
    return STRATA_ERR_ARG;
  if (shared_kind != K_Q4_K || pairs > 65535 || shared_rows > INT32_MAX / 2) return STRATA_ERR_SHAPE;
  p.blocks[0] = (const uint8_t*)gate_blocks;
  p.blocks[1] = (const uint8_t*)up_blocks;
  p.out[0] = out_gate;
  p.out[1] = out_up;
  p.glu_out = out_h;
  p.idx = idx;
  p.x = x;
  p.mat_bytes = rows * (int64_t)p.row_bytes;
  p.experts = experts;
  p.src_rows = (int)rows;
  p.rows = (int)rows;
  p.cols = (int)cols;
  p.pairs = (int)pairs;
  p.share = (int)pairs;  // one token
  p.mode = MODE_EXPERT;
  p.shared[0] = (const uint8_t*)shared_gate;
  p.shared[1] = (const uint8_t*)shared_up;
  p.shared_out = shared_h;
  p.shared_gu[0] = shared_g;
  p.shared_gu[1] = shared_u;
  p.shared_rows = (int)shared_rows;
  p.shared_row_bytes = s_row_bytes;
  p.route_logits = logits;
  p.route_idx = idx_out;
  p.route_w = w_out;
  p.route_extra = extra_out;
  p.route_rows = (int)logit_rows;
  p.route_experts = (int)route_experts;
  return launch_by_kind(kind, p, x_dtype, x_dtype, false, (int)pairs, 2, (hipStream_t)stream);
}

extern "C" {

int strata_abi_version(void) { return 6; }

int strata_block_info(int kind, int* per_block, int* block_bytes) {
  return strata_kind_info(kind, per_block, block_bytes) ? STRATA_ERR_KIND : STRATA_OK;
}

int strata_dequant(int kind, const void* blocks, int64_t n_mats, int64_t rows, int64_t cols, void* out,
                   int out_dtype, void* stream) {
  int row_bytes = 0;
  int rc = block_shape(kind, rows, cols, &row_bytes);
  if (rc) return rc;
  if (n_mats < 0) return STRATA_ERR_SHAPE;
  if (out_dtype != DT_F32 && out_dtype != DT_F16) return STRATA_ERR_DTYPE;
  const int64_t runs_total = n_mats * rows * (cols / 32);
  if (runs_total == 0) return STRATA_OK;
  if (!blocks || !out) return STRATA_ERR_ARG;
  if ((runs_total + 255) / 256 > INT32_MAX) return STRATA_ERR_SHAPE;
  return dequant_by_kind(kind, (const uint8_t*)blocks, runs_total, (int)(cols / 32), row_bytes, out, out_dtype,
                         (hipStream_t)stream);
}

int strata_expert_matvec(int kind, const void* blocks, int64_t experts, int64_t rows, int64_t cols,
                         const uint32_t* idx, int64_t pairs, const void* x, int x_dtype, int64_t share, void* out,
                         void* stream) {
  return expert_common(kind, blocks, nullptr, experts, rows, cols, idx, pairs, x, nullptr, x_dtype, share, out,
                       nullptr, false, stream);
}

int strata_expert_matvec2(int kind, const void* blocks_a, const void* blocks_b, int64_t experts, int64_t rows,
                          int64_t cols, const uint32_t* idx, int64_t pairs, const void* x, int x_dtype, int64_t share,
                          void* out_a, void* out_b, void* stream) {
  if (!blocks_b && pairs > 0 && rows > 0) return STRATA_ERR_ARG;
  return expert_common(kind, blocks_a, blocks_b, experts, rows, cols, idx, pairs, x, nullptr, x_dtype, share, out_a,
                       out_b, false, stream);
}

int strata_expert_gate_up_swiglu(int kind, const void* gate_blocks, const void* up_blocks, int64_t experts,
                                 int64_t rows, int64_t cols, const uint32_t* idx, int64_t pairs, const void* x,
                                 int x_dtype, int64_t share, void* out_gate, void* out_up, void* out_h, void* stream) {
  if ((!up_blocks || !out_h) && pairs > 0 && rows > 0) return STRATA_ERR_ARG;
  return expert_common(kind, gate_blocks, up_blocks, experts, rows, cols, idx, pairs, x, nullptr, x_dtype, share,
                       out_gate, out_up, false, stream, out_h);
}

int strata_expert_gate_up_swiglu_shared(int kind, const void* gate_blocks, const void* up_blocks, int64_t experts,
                                        int64_t rows, int64_t cols, const uint32_t* idx, int64_t pairs,
                                        const void* x, int x_dtype, void* out_gate, void* out_up, void* out_h,
                                        int shared_kind, const void* shared_gate, const void* shared_up,
                                        int64_t shared_rows, void* shared_h, void* shared_g, void* shared_u,
                                        void* stream) {
  if (!idx) return STRATA_ERR_ARG;
  return gate_up_shared(kind, gate_blocks, up_blocks, experts, rows, cols, idx, pairs, x, x_dtype, out_gate, out_up,
                        out_h, shared_kind, shared_gate, shared_up, shared_rows, shared_h, shared_g, shared_u, nullptr,
                        0, 0, nullptr, nullptr, nullptr, stream);
}

int strata_moe_gate_up_swiglu_shared(int kind, const void* gate_blocks, const void* up_blocks, int64_t experts,
                                     int64_t rows, int64_t cols, const float* logits, int64_t logit_rows,
                                     int64_t pairs, const void* x, int x_dtype, void* out_h, uint32_t* idx_out,
                                     float* w_out, int shared_kind, const void* shared_gate, const void* shared_up,
                                     int64_t shared_rows, void* shared_h, void* extra_out, void* stream) {
  if (!logits || !idx_out || !w_out) return STRATA_ERR_ARG;
  if (logit_rows < experts || experts > 256 || pairs > 64 || pairs > experts) return STRATA_ERR_SHAPE;
  return gate_up_shared(kind, gate_blocks, up_blocks, experts, rows, cols, idx_out, pairs, x, x_dtype, nullptr,
                        nullptr, out_h, shared_kind, shared_gate, shared_up, shared_rows, shared_h, nullptr, nullptr,
                        logits, logit_rows, experts, idx_out, w_out, extra_out, stream);
}

int strata_expert_matvec_shared(int kind, const void* blocks, int64_t experts, int64_t rows, int64_t cols,
                                const uint32_t* idx, int64_t pairs, const void* x, int x_dtype, void* out,
                                int shared_kind, const void* shared_blocks, int64_t shared_rows, const void* shared_x,
                                void* shared_out, void* stream) {
  MatvecParams p = {};
  int rc = block_shape(kind, rows, cols, &p.row_bytes);
  if (rc) return rc;
  int s_row_bytes = 0;
  rc = block_shape(shared_kind, shared_rows, cols, &s_row_bytes);
  if (rc) return rc;
  if (x_dtype != DT_F16) return STRATA_ERR_DTYPE;
  if (pairs < 1 || experts < 1 || experts > INT32_MAX || shared_rows < 1) return STRATA_ERR_ARG;
  if (rows == 0) return STRATA_ERR_SHAPE;  // no routed launch to carry the shared expert: the two calls apart
  if (!blocks || !idx || !x || !out || !shared_blocks || !shared_x || !shared_out) return STRATA_ERR_ARG;
  if (shared_kind != K_Q4_K || pairs > 65535 || shared_rows > INT32_MAX / 2) return STRATA_ERR_SHAPE;
  p.blocks[0] = (const uint8_t*)blocks;
  p.out[0] = out;
  p.idx = idx;
  p.x = x;
  p.mat_bytes = rows * (int64_t)p.row_bytes;
  p.experts = experts;
  p.src_rows = (int)rows;
  p.rows = (int)rows;
  p.cols = (int)cols;
  p.pairs = (int)pairs;
  p.share = 1;  // each pair its own token (its h)
  p.mode = MODE_EXPERT;
  p.shared[0] = (const uint8_t*)shared_blocks;
  p.shared_x = shared_x;
  p.shared_out = shared_out;
  p.shared_rows = (int)shared_rows;
  p.shared_row_bytes = s_row_bytes;
  return launch_by_kind(kind, p, x_dtype, x_dtype, false, (int)pairs, 1, (hipStream_t)stream);
}

int strata_expert_matvec_swiglu(int kind, const void* blocks, int64_t experts, int64_t rows, int64_t cols,
                                const uint32_t* idx, int64_t pairs, const void* gate, const void* up, int act_dtype,
                                void* out, void* stream) {
  return expert_common(kind, blocks, nullptr, experts, rows, cols, idx, pairs, gate, up, act_dtype, 1, out, nullptr,
                       true, stream);
}

int strata_expert_matvec_ptrs(int kind, const void* const* per_pair, int64_t rows, int64_t cols, int64_t pairs,
                              const void* x, int x_dtype, int64_t share, void* out, void* stream) {
  MatvecParams p = {};
  int rc = block_shape(kind, rows, cols, &p.row_bytes);
  if (rc) return rc;
  if (!valid_dtype(x_dtype)) return STRATA_ERR_DTYPE;
  if (pairs < 0) return STRATA_ERR_ARG;
  if (pairs == 0 || rows == 0) return STRATA_OK;
  if (!per_pair || !x || !out) return STRATA_ERR_ARG;
  if (share < 1 || pairs % share) return STRATA_ERR_ARG;
  if (pairs > 65535 || cols / 32 > 256) return STRATA_ERR_SHAPE;
  p.ptrs = (const uint8_t* const*)per_pair;
  p.out[0] = out;
  p.x = x;
  p.mat_bytes = rows * (int64_t)p.row_bytes;
  p.src_rows = (int)rows;
  p.rows = (int)rows;
  p.cols = (int)cols;
  p.pairs = (int)pairs;
  p.share = (int)share;
  p.mode = MODE_PTRS;
  return launch_by_kind(kind, p, x_dtype, x_dtype, false, (int)pairs, 1, (hipStream_t)stream);
}

int strata_dense_matvec(int kind, const void* blocks, int64_t rows, int64_t cols, const void* x, int64_t tokens,
                        int x_dtype, void* out, int out_dtype, const uint32_t* row_ids, int64_t n_ids, void* stream) {
  MatvecParams p = {};
  int rc = block_shape(kind, rows, cols, &p.row_bytes);
  if (rc) return rc;
  if (!valid_dtype(x_dtype) || !valid_dtype(out_dtype)) return STRATA_ERR_DTYPE;
  if (tokens < 0 || (row_ids && n_ids < 0)) return STRATA_ERR_ARG;
  const int64_t out_rows = row_ids ? n_ids : rows;
  if (tokens == 0 || out_rows == 0) return STRATA_OK;
  if (!blocks || !x || !out) return STRATA_ERR_ARG;
  if (tokens > 65535 || out_rows > INT32_MAX / 2 || cols / 32 > 256) return STRATA_ERR_SHAPE;
  if (out_dtype != x_dtype && out_dtype != DT_F32) return STRATA_ERR_DTYPE;
  p.blocks[0] = (const uint8_t*)blocks;
  p.out[0] = out;
  p.row_ids = row_ids;
  p.x = x;
  p.mat_bytes = rows * (int64_t)p.row_bytes;
  p.src_rows = (int)rows;
  p.rows = (int)out_rows;
  p.cols = (int)cols;
  p.tokens = (int)tokens;
  p.mode = MODE_DENSE;
  return launch_by_kind(kind, p, x_dtype, out_dtype, false, 1, 1, (hipStream_t)stream);
}

}  // extern "C"
