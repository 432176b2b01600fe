// Q3_K held as planes (strata_mlx/blocks.py:397-512): a tensor's 110-byte blocks rearranged once into aligned
// arrays of their parts, the same weights.
//
//   hm  uint32 [blocks][8]   the block's 32 high-bit bytes (bit r of byte i: weight i of run r is >= 0 ... < 4)
//   qs  uint32 [blocks][16]  the 64 bytes of 2-bit values (half n of the block: words 8n .. 8n + 7)
//   sc  int8   [blocks][16]  the sixteen 6-bit scales, decoded, less 32
//   dd  f16    [blocks]      d
//
// 114 bytes a block where the file has 110. Weight i = 4 w + k (k < 4) of run rr = 4 n + j of a block is
// d * sc[2 rr + (w >= 4)] * (((qs[8 n + w] >> (8 k + 2 j)) & 3) - ((hm[w] >> (8 k + rr)) & 1 ? 0 : 4)).
//
//   q3k_planes_kernel   one thread a block: the planes from the file's block (strata_mlx/blocks.py:403-414)
//   q3k_window_kernel   out[t, r] = W[r, :] . x[t, :] for up to 8 tokens (48 KB of activations, staged in LDS
//                       once a workgroup): P lanes a row, lane `part` taking half blocks part, part + P, ...; a
//                       run's two halves of 16 weights summed apart (four-weight dot products in order), then
//                       d * sc of each added to the lane's sums; the row's lanes by a butterfly. P depends on the
//                       tensor's shape only, so a token gets the same bits alone as in a window
//                       (strata_mlx/blocks.py:425-461, 482-501).
//   q3k_dequant_kernel  one thread a run of 32: (d * sc) * value, exact in float32 (blocks.py:464-479, 504-512).
// The window kernel is HBM-bound: 114 bytes per 256 weights per row, read once for every token of the window.
#include <algorithm>

#include "common.h"
#include "decode.h"

namespace {

constexpr int kPThreads = 256;
constexpr int kPMaxTokens = 8;
constexpr size_t kPMaxXBytes = 48 * 1024;  // a launch's activations, staged in LDS

__global__ __launch_bounds__(kPThreads) void q3k_planes_kernel(const uint8_t* __restrict__ blocks, int64_t n_blocks,
                                                               uint32_t* __restrict__ hm, uint32_t* __restrict__ qs,
                                                               int8_t* __restrict__ sc, f16* __restrict__ dd) {
  const int64_t blk = (int64_t)blockIdx.x * kPThreads + threadIdx.x;
  if (blk >= n_blocks) return;
  const uint8_t* b = blocks + blk * 110;  // hmask[32] @0, qs[64] @32, scales[12] @96, d @108
#pragma unroll
  for (int w = 0; w < 8; ++w) hm[blk * 8 + w] = strata_u32_at(b + 4 * w);
#pragma unroll
  for (int w = 0; w < 16; ++w) qs[blk * 16 + w] = strata_u32_at(b + 32 + 4 * w);
#pragma unroll
  for (int k = 0; k < 16; ++k) sc[blk * 16 + k] = (int8_t)(int)strata_q3k_scale(b + 96, (uint32_t)k);
  dd[blk] = __builtin_bit_cast(f16, (uint16_t)strata_u16_at(b + 108));
}

__device__ __forceinline__ float q3k_value(uint32_t qw, uint32_t hw, int k, int j, int rr) {
  return (float)((int)((qw >> (8 * k + 2 * j)) & 3u) - (((hw >> (8 * k + rr)) & 1u) ? 0 : 4));
}

struct PlanesParams {
  const uint32_t* hm;
  const uint32_t* qs;
  const int8_t* sc;
  const f16* dd;
  const void* x;
  void* out;
  int rows, cols, tokens, per_row;
};

// A workgroup: 256 / P rows, its tokens' activations staged once in LDS in their own type.
template <typename XT>
__global__ __launch_bounds__(kPThreads) void q3k_window_kernel(PlanesParams p) {
  extern __shared__ __attribute__((aligned(16))) unsigned char xs_raw[];
  XT* xs = reinterpret_cast<XT*>(xs_raw);  // (tokens, cols)
  const int tid = threadIdx.x;
  {
    const int n16 = p.tokens * p.cols * (int)sizeof(XT) / 16;
    const u32x4* src = reinterpret_cast<const u32x4*>(p.x);
    u32x4* dst = reinterpret_cast<u32x4*>(xs_raw);
    for (int i = tid; i < n16; i += kPThreads) dst[i] = src[i];
  }
  __syncthreads();
  const int P = p.per_row;
  const int part = tid % P;
  const int r = blockIdx.x * (kPThreads / P) + tid / P;
  const bool live = r < p.rows;
  const int row = live ? r : p.rows - 1;  // lanes of a row past the end keep to the shuffles, write nothing
  const int blocks = p.cols / 256;
  float sum[kPMaxTokens];
#pragma unroll
  for (int t = 0; t < kPMaxTokens; ++t) sum[t] = 0.0f;
  for (int h = part; h < 2 * blocks; h += P) {  // half a block, 128 weights, at a time
    const int64_t blk = (int64_t)row * blocks + h / 2;
    const int n = h % 2;
    const u32x4* hm4 = reinterpret_cast<const u32x4*>(p.hm + blk * 8);
    const u32x4* qs4 = reinterpret_cast<const u32x4*>(p.qs + blk * 16 + 8 * n);
    const u32x4 h0 = hm4[0], h1 = hm4[1], q0 = qs4[0], q1 = qs4[1];
    const uint32_t hw[8] = {h0[0], h0[1], h0[2], h0[3], h1[0], h1[1], h1[2], h1[3]};
    const uint32_t qw[8] = {q0[0], q0[1], q0[2], q0[3], q1[0], q1[1], q1[2], q1[3]};
    const u32x2 scw = *reinterpret_cast<const u32x2*>(p.sc + blk * 16 + 8 * n);  // the half's eight scales
    const float d = (float)p.dd[blk];
    const int base = (h / 2) * 256 + 128 * n;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int rr = 4 * n + j;
      float acc0[kPMaxTokens], acc1[kPMaxTokens];
#pragma unroll
      for (int t = 0; t < kPMaxTokens; ++t) acc0[t] = acc1[t] = 0.0f;
#pragma unroll
      for (int w = 0; w < 8; ++w) {
        float v[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) v[k] = q3k_value(qw[w], hw[w], k, j, rr);
        const int xi = base + 32 * j + 4 * w;
#pragma unroll
        for (int t = 0; t < kPMaxTokens; ++t) {
          if (t < p.tokens) {
            const XT* xt = xs + t * p.cols + xi;
            float dot = v[0] * to_f32(xt[0]);
            dot = __fmaf_rn(v[1], to_f32(xt[1]), dot);
            dot = __fmaf_rn(v[2], to_f32(xt[2]), dot);
            dot = __fmaf_rn(v[3], to_f32(xt[3]), dot);
            if (w < 4)
              acc0[t] += dot;
            else
              acc1[t] += dot;
          }
        }
      }
      const uint32_t sw = scw[j / 2] >> (16 * (j % 2));  // scales 2 rr, 2 rr + 1 of the half
      const float s0 = d * (float)(int8_t)(sw & 255u), s1 = d * (float)(int8_t)((sw >> 8) & 255u);
#pragma unroll
      for (int t = 0; t < kPMaxTokens; ++t) sum[t] += __fmaf_rn(s0, acc0[t], s1 * acc1[t]);
    }
  }
#pragma unroll
  for (int t = 0; t < kPMaxTokens; ++t) {
    if (t < p.tokens) {
      float total = sum[t];
      for (int k = 1; k < P; k <<= 1) total += __shfl_xor(total, k, P);
      if (live && part == 0) reinterpret_cast<XT*>(p.out)[(int64_t)t * p.rows + r] = from_f32<XT>(total);
    }
  }
}

template <typename OT>
__global__ __launch_bounds__(kPThreads) void q3k_dequant_kernel(PlanesParams p, int64_t n_runs) {
  const int64_t run = (int64_t)blockIdx.x * kPThreads + threadIdx.x;  // (row, block, run)
  if (run >= n_runs) return;
  const int rr = (int)(run % 8);
  const int64_t blk = run / 8;
  const int n = rr / 4, j = rr % 4;
  const float d = (float)p.dd[blk];
  const float s0 = d * (float)p.sc[blk * 16 + 2 * rr], s1 = d * (float)p.sc[blk * 16 + 2 * rr + 1];
  OT* o = reinterpret_cast<OT*>(p.out) + blk * 256 + 32 * rr;
#pragma unroll
  for (int w = 0; w < 8; ++w) {
    const uint32_t qw = p.qs[blk * 16 + 8 * n + w], hw = p.hm[blk * 8 + w];
#pragma unroll
    for (int k = 0; k < 4; ++k) o[4 * w + k] = from_f32<OT>((w < 4 ? s0 : s1) * q3k_value(qw, hw, k, j, rr));
  }
}

int planes_shape(int64_t rows, int64_t cols) {
  if (rows < 0 || cols < 0) return STRATA_ERR_ARG;
  if (cols % 256 || rows > (1 << 24) || cols > (1 << 20) || rows * (cols / 256) > ((int64_t)1 << 31))
    return STRATA_ERR_SHAPE;
  return STRATA_OK;
}

}  // namespace

extern "C" {

int strata_q3k_planes(const void* blocks, int64_t rows, int64_t cols, uint32_t* hm, uint32_t* qs, int8_t* sc,
                      void* dd, void* stream) {
  int rc = planes_shape(rows, cols);
  if (rc) return rc;
  if (rows == 0 || cols == 0) return STRATA_OK;
  if (!blocks || !hm || !qs || !sc || !dd) return STRATA_ERR_ARG;
  const int64_t n = rows * (cols / 256);
  hipLaunchKernelGGL(q3k_planes_kernel, dim3((unsigned)((n + kPThreads - 1) / kPThreads)), dim3(kPThreads), 0,
                     (hipStream_t)stream, (const uint8_t*)blocks, n, hm, qs, sc, (f16*)dd);
  STRATA_CHECK_LAUNCH();
  return STRATA_OK;
}

int strata_q3k_planes_window(const uint32_t* hm, const uint32_t* qs, const int8_t* sc, const void* dd, int64_t rows,
                             int64_t cols, const void* x, int64_t tokens, int x_dtype, int per_row, void* out,
                             void* stream) {
  int rc = planes_shape(rows, cols);
  if (rc) return rc;
  if (tokens < 0) return STRATA_ERR_ARG;
  if (rows == 0 || tokens == 0) return STRATA_OK;
  if (!hm || !qs || !sc || !dd || !x || !out) return STRATA_ERR_ARG;
  if (per_row < 1 || per_row > 64 || (per_row & (per_row - 1))) return STRATA_ERR_ARG;
  if (x_dtype != DT_F32 && x_dtype != DT_F16 && x_dtype != DT_BF16) return STRATA_ERR_DTYPE;
  const size_t x_bytes = (size_t)tokens * (size_t)cols * (x_dtype == DT_F32 ? 4 : 2);
  if (tokens > kPMaxTokens || x_bytes > kPMaxXBytes) return STRATA_ERR_SHAPE;
  PlanesParams p = {hm, qs, sc, (const f16*)dd, x, out, (int)rows, (int)cols, (int)tokens, per_row};
  const int64_t threads = rows * per_row;
  const dim3 grid((unsigned)((threads + kPThreads - 1) / kPThreads));
  hipStream_t s = (hipStream_t)stream;
  if (x_dtype == DT_F32)
    hipLaunchKernelGGL(q3k_window_kernel<float>, grid, dim3(kPThreads), x_bytes, s, p);
  else if (x_dtype == DT_F16)
    hipLaunchKernelGGL(q3k_window_kernel<f16>, grid, dim3(kPThreads), x_bytes, s, p);
  else
    hipLaunchKernelGGL(q3k_window_kernel<bf16_t>, grid, dim3(kPThreads), x_bytes, s, p);
  STRATA_CHECK_LAUNCH();
  return STRATA_OK;
}

int strata_q3k_planes_dequant(const uint32_t* hm, const uint32_t* qs, const int8_t* sc, const void* dd, int64_t rows,
                              int64_t cols, void* out, int out_dtype, void* stream) {
  int rc = planes_shape(rows, cols);
  if (rc) return rc;
  if (rows == 0 || cols == 0) return STRATA_OK;
  if (!hm || !qs || !sc || !dd || !out) return STRATA_ERR_ARG;
  PlanesParams p = {hm, qs, sc, (const f16*)dd, nullptr, out, (int)rows, (int)cols, 0, 1};
  const int64_t runs = rows * (cols / 32);
  const dim3 grid((unsigned)((runs + kPThreads - 1) / kPThreads));
  hipStream_t s = (hipStream_t)stream;
  if (out_dtype == DT_F32)
    hipLaunchKernelGGL(q3k_dequant_kernel<float>, grid, dim3(kPThreads), 0, s, p, runs);
  else if (out_dtype == DT_F16)
    hipLaunchKernelGGL(q3k_dequant_kernel<f16>, grid, dim3(kPThreads), 0, s, p, runs);
  else
    return STRATA_ERR_DTYPE;
  STRATA_CHECK_LAUNCH();
  return STRATA_OK;
}

}  // extern "C"
