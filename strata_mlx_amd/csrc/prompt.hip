// C-ABI entry points of a prompt's expert products in tiles (declared in include/strata_gfx950.h): gate and up with
// the SwiGLU in one launch, down written straight to the pairs, and the scaling of 16-bit rows into float16.
// Kernels in prompt_impl.h (instantiated per type by gemm_kind.hip).
#include "gemm_impl.h"
#include "prompt_impl.h"

namespace strata_prompt {
#define STRATA_DECLARE(K) int prompt_launch_##K(PromptParams&, int, int, hipStream_t);
STRATA_DECLARE(18)
STRATA_DECLARE(21)
STRATA_DECLARE(42)
#undef STRATA_DECLARE

namespace {

constexpr int kRowThreads = 256;

// One workgroup a row: its largest magnitude, then the row divided by the power of two that puts it in
// [2^14, 2^15), rounded to float16 (exact for every value within 2^31 of the largest).
template <typename AT>
__global__ __launch_bounds__(kRowThreads) void rows_to_f16_kernel(const AT* a, int cols, f16* out, uint32_t* row_max) {
  __shared__ uint32_t wmax[kRowThreads / 64];
  const int64_t r = blockIdx.x;
  const AT* src = a + r * cols;
  uint32_t m = 0;
  for (int c = threadIdx.x; c < cols; c += kRowThreads) m = max(m, __float_as_uint(to_f32(src[c])) & 0x7fffffffu);
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) m = max(m, (uint32_t)__shfl_xor((int)m, d));
  if ((threadIdx.x & 63) == 0) wmax[threadIdx.x >> 6] = m;
  __syncthreads();
#pragma unroll
  for (int w = 0; w < kRowThreads / 64; ++w) m = max(m, wmax[w]);
  const int ex = row_exponent(m);
  f16* dst = out + r * cols;
  for (int c = threadIdx.x; c < cols; c += kRowThreads) dst[c] = from_f32<f16>(__builtin_ldexpf(to_f32(src[c]), -ex));
  if (threadIdx.x == 0) row_max[r] = m;
}

// rows_to_f16 for 16-bit rows of at most 8192 values, a multiple of 8: the row read once, 16 bytes (8 values) a
// piece and up to CH pieces a thread held in registers between the row's maximum and the scaled stores.
template <typename AT, int CH>
__global__ __launch_bounds__(kRowThreads) void rows_to_f16_vec_kernel(const AT* a, int cols, f16* out,
                                                                      uint32_t* row_max) {
  static_assert(sizeof(AT) == 2, "16-bit rows");
  __shared__ uint32_t wmax[kRowThreads / 64];
  const int64_t r = blockIdx.x;
  const int pieces = cols / 8;
  const u32x4* src = reinterpret_cast<const u32x4*>(a + r * cols);
  u32x4 v[CH];
  uint32_t m = 0;
#pragma unroll
  for (int k = 0; k < CH; ++k) {
    const int c = threadIdx.x + k * kRowThreads;
    v[k] = c < pieces ? src[c] : u32x4{0u, 0u, 0u, 0u};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const AT lo = __builtin_bit_cast(AT, (uint16_t)(v[k][i] & 0xffffu));
      const AT hi = __builtin_bit_cast(AT, (uint16_t)(v[k][i] >> 16));
      m = max(m, __float_as_uint(to_f32(lo)) & 0x7fffffffu);
      m = max(m, __float_as_uint(to_f32(hi)) & 0x7fffffffu);
    }
  }
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) m = max(m, (uint32_t)__shfl_xor((int)m, d));
  if ((threadIdx.x & 63) == 0) wmax[threadIdx.x >> 6] = m;
  __syncthreads();
#pragma unroll
  for (int w = 0; w < kRowThreads / 64; ++w) m = max(m, wmax[w]);
  const int ex = row_exponent(m);
  u32x4* dst = reinterpret_cast<u32x4*>(out + r * cols);
#pragma unroll
  for (int k = 0; k < CH; ++k) {
    const int c = threadIdx.x + k * kRowThreads;
    if (c < pieces) {
      uint32_t o[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const AT lo = __builtin_bit_cast(AT, (uint16_t)(v[k][i] & 0xffffu));
        const AT hi = __builtin_bit_cast(AT, (uint16_t)(v[k][i] >> 16));
        o[i] = (uint32_t)__builtin_bit_cast(uint16_t, from_f32<f16>(__builtin_ldexpf(to_f32(lo), -ex))) |
               ((uint32_t)__builtin_bit_cast(uint16_t, from_f32<f16>(__builtin_ldexpf(to_f32(hi), -ex))) << 16);
      }
      dst[c] = u32x4{o[0], o[1], o[2], o[3]};
    }
  }
  if (threadIdx.x == 0) row_max[r] = m;
}

// The products of rows scaled by rows_to_f16 scaled back, out[r, c] = c[r, c] * 2^e(r), rounded once to OT: four
// values a thread (one 16-byte load where a row's length is a multiple of four), a row of blocks a row.
template <typename OT>
__global__ __launch_bounds__(256) void rows_from_f32_kernel(const float* c, int cols, const uint32_t* row_max,
                                                            OT* out) {
  const int64_t r = blockIdx.y;
  const int ex = row_exponent(row_max[r]);
  const int i = (blockIdx.x * 256 + threadIdx.x) * 4;
  if (i >= cols) return;
  const float* src = c + r * cols + i;
  OT* dst = out + r * cols + i;
  if ((cols & 3) == 0) {
    const float4 v = *reinterpret_cast<const float4*>(src);
    dst[0] = from_f32<OT>(__builtin_ldexpf(v.x, ex));
    dst[1] = from_f32<OT>(__builtin_ldexpf(v.y, ex));
    dst[2] = from_f32<OT>(__builtin_ldexpf(v.z, ex));
    dst[3] = from_f32<OT>(__builtin_ldexpf(v.w, ex));
  } else {
    for (int j = 0; j < 4 && i + j < cols; ++j) dst[j] = from_f32<OT>(__builtin_ldexpf(src[j], ex));
  }
}

// Rows of y for the pairs naming no expert: NaN, as every matvec gives them.
template <typename OT>
__global__ __launch_bounds__(256) void nan_rows_kernel(const uint32_t* idx, int64_t experts, int cols, OT* y) {
  const int64_t p = blockIdx.x;
  if (idx[p] < (uint64_t)experts) return;
  for (int c = threadIdx.x; c < cols; c += 256) y[p * cols + c] = from_f32<OT>(__builtin_nanf(""));
}

int dispatch(int kind, PromptParams& p, int mode, int out_dtype, hipStream_t s) {
  switch (kind) {
    case 18: return prompt_launch_18(p, mode, out_dtype, s);
    case 21: return prompt_launch_21(p, mode, out_dtype, s);
    case 42: return prompt_launch_42(p, mode, out_dtype, s);
    default: return STRATA_ERR_KIND;
  }
}

int common_checks(int kind, int64_t experts, int64_t rows, int64_t cols, int64_t n_tiles, int64_t tile, int dtype) {
  if (!prompt_takes(kind, cols)) {
    int per = 0, bb = 0;
    if (strata_kind_info(kind, &per, &bb)) return STRATA_ERR_KIND;
    return cols > 0 && cols % per == 0 ? STRATA_ERR_KIND : STRATA_ERR_SHAPE;
  }
  if (rows < 0 || rows > (1 << 24) || cols > (1 << 20)) return STRATA_ERR_SHAPE;
  int per = 0, bb = 0;
  strata_kind_info(kind, &per, &bb);
  if (rows * (cols / per * bb) >= (int64_t(1) << 32)) return STRATA_ERR_SHAPE;  // row offsets in a matrix are 32-bit
  if (dtype != DT_F16 && dtype != DT_BF16) return STRATA_ERR_DTYPE;
  if (tile != 16 || n_tiles < 0 || n_tiles > (1 << 24) || experts < 0) return STRATA_ERR_ARG;
  return STRATA_OK;
}

void fill_shape(PromptParams& p, int kind, int64_t experts, int64_t rows, int64_t cols, int64_t n_tiles) {
  int per = 0, bb = 0;
  strata_kind_info(kind, &per, &bb);
  p.experts = experts;
  p.rows = (int)rows;
  p.cols = (int)cols;
  p.row_bytes = (int)(cols / per * bb);
  p.mat_bytes = rows * (int64_t)p.row_bytes;
  p.n_tiles = (int)n_tiles;
}

}  // namespace
}  // namespace strata_prompt

using namespace strata_prompt;

extern "C" int strata_rows_from_f32(const float* c, int64_t rows, int64_t cols, const uint32_t* row_max, int out_dtype,
                                    void* out, void* stream) {
  if (rows < 0 || cols < 0 || cols > (1 << 28) || rows > 65535) return STRATA_ERR_SHAPE;
  if (rows == 0 || cols == 0) return STRATA_OK;
  if (!c || !row_max || !out) return STRATA_ERR_ARG;
  hipStream_t s = (hipStream_t)stream;
  const dim3 grid((unsigned)((cols + 1023) / 1024), (unsigned)rows);
  if (out_dtype == DT_BF16)
    hipLaunchKernelGGL((rows_from_f32_kernel<bf16_t>), grid, dim3(256), 0, s, c, (int)cols, row_max, (bf16_t*)out);
  else if (out_dtype == DT_F16)
    hipLaunchKernelGGL((rows_from_f32_kernel<f16>), grid, dim3(256), 0, s, c, (int)cols, row_max, (f16*)out);
  else if (out_dtype == DT_F32)
    hipLaunchKernelGGL((rows_from_f32_kernel<float>), grid, dim3(256), 0, s, c, (int)cols, row_max, (float*)out);
  else
    return STRATA_ERR_DTYPE;
  STRATA_CHECK_LAUNCH();
  return STRATA_OK;
}

extern "C" int strata_rows_to_f16(const void* a, int64_t rows, int64_t cols, int a_dtype, void* out, uint32_t* row_max,
                                  void* stream) {
  if (rows < 0 || cols < 0 || cols > (1 << 24) || rows > 0x7fffffff) return STRATA_ERR_SHAPE;
  if (rows == 0 || cols == 0) return STRATA_OK;
  if (!a || !out || !row_max) return STRATA_ERR_ARG;
  hipStream_t s = (hipStream_t)stream;
  // 16-bit rows of at most 8192 values, a multiple of 8, at 16-byte aligned addresses: read once, 16 bytes a load
  const bool vec = (a_dtype == DT_BF16 || a_dtype == DT_F16) && cols % 8 == 0 && cols <= 8 * 4 * kRowThreads &&
                   ((uintptr_t)a & 15) == 0 && ((uintptr_t)out & 15) == 0;
  if (vec) {
    const int ch = (int)((cols / 8 + kRowThreads - 1) / kRowThreads);  // pieces a thread: 1 to 4
    auto go = [&](auto tag, auto chc) {
      typedef decltype(tag) AT;
      hipLaunchKernelGGL((rows_to_f16_vec_kernel<AT, decltype(chc)::value>), dim3((unsigned)rows), dim3(kRowThreads),
                         0, s, (const AT*)a, (int)cols, (f16*)out, row_max);
    };
    auto by_ch = [&](auto tag) {
      switch (ch) {
        case 1: go(tag, std::integral_constant<int, 1>()); break;
        case 2: go(tag, std::integral_constant<int, 2>()); break;
        case 3: go(tag, std::integral_constant<int, 3>()); break;
        default: go(tag, std::integral_constant<int, 4>()); break;
      }
    };
    if (a_dtype == DT_BF16)
      by_ch(bf16_t{});
    else
      by_ch(f16{});
    STRATA_CHECK_LAUNCH();
    return STRATA_OK;
  }
  if (a_dtype == DT_BF16)
    hipLaunchKernelGGL((rows_to_f16_kernel<bf16_t>), dim3((unsigned)rows), dim3(kRowThreads), 0, s,
                       (const bf16_t*)a, (int)cols, (f16*)out, row_max);
  else if (a_dtype == DT_F16)
    hipLaunchKernelGGL((rows_to_f16_kernel<f16>), dim3((unsigned)rows), dim3(kRowThreads), 0, s, (const f16*)a,
                       (int)cols, (f16*)out, row_max);
  else if (a_dtype == DT_F32)
    hipLaunchKernelGGL((rows_to_f16_kernel<float>), dim3((unsigned)rows), dim3(kRowThreads), 0, s, (const float*)a,
                       (int)cols, (f16*)out, row_max);
  else
    return STRATA_ERR_DTYPE;
  STRATA_CHECK_LAUNCH();
  return STRATA_OK;
}

extern "C" int strata_prompt_gate_up_swiglu(int kind, const void* gate, const void* up, int64_t experts, int64_t rows,
                                            int64_t cols, const void* x, const uint32_t* x_max, const uint32_t* token,
                                            const uint32_t* tile_expert, int64_t n_tiles, int64_t tile, void* h,
                                            int h_dtype, void* stream) {
  const int rc = common_checks(kind, experts, rows, cols, n_tiles, tile, h_dtype);
  if (rc) return rc;
  if (n_tiles == 0 || rows == 0) return STRATA_OK;
  if (!gate || !up || !x || !token || !tile_expert || !h) return STRATA_ERR_ARG;
  PromptParams p = {};
  fill_shape(p, kind, experts, rows, cols, n_tiles);
  p.blocks[0] = (const uint8_t*)gate;
  p.blocks[1] = (const uint8_t*)up;
  p.a = (const f16*)x;
  p.a_row = token;
  p.a_max = x_max;
  p.tile_expert = tile_expert;
  p.out = h;
  return dispatch(kind, p, PM_GLU, h_dtype, (hipStream_t)stream);
}

extern "C" int strata_prompt_down(int kind, const void* blocks, int64_t experts, int64_t rows, int64_t cols,
                                  const void* h, const uint32_t* h_max, const uint32_t* tile_expert, int64_t n_tiles,
                                  int64_t tile, const uint32_t* slot_pair, const uint32_t* idx, int64_t pairs, void* y,
                                  int y_dtype, void* stream) {
  const int rc = common_checks(kind, experts, rows, cols, n_tiles, tile, y_dtype);
  if (rc) return rc;
  if (pairs < 0 || pairs > 0x7fffffff) return STRATA_ERR_ARG;
  if (pairs == 0 || rows == 0) return STRATA_OK;
  if (!blocks || !idx || !y || (n_tiles > 0 && (!h || !tile_expert || !slot_pair))) return STRATA_ERR_ARG;
  hipStream_t s = (hipStream_t)stream;
  if (y_dtype == DT_F16)
    hipLaunchKernelGGL((nan_rows_kernel<f16>), dim3((unsigned)pairs), dim3(256), 0, s, idx, experts, (int)rows, (f16*)y);
  else
    hipLaunchKernelGGL((nan_rows_kernel<bf16_t>), dim3((unsigned)pairs), dim3(256), 0, s, idx, experts, (int)rows,
                       (bf16_t*)y);
  STRATA_CHECK_LAUNCH();
  if (n_tiles == 0) return STRATA_OK;
  PromptParams p = {};
  fill_shape(p, kind, experts, rows, cols, n_tiles);
  p.blocks[0] = (const uint8_t*)blocks;
  p.a = (const f16*)h;
  p.a_max = h_max;
  p.tile_expert = tile_expert;
  p.slot_pair = slot_pair;
  p.out = y;
  return dispatch(kind, p, PM_SCATTER, y_dtype, s);
}
