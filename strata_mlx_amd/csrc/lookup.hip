// Q2_0 products from a table of sums (strata_mlx/blocks.py:697-928), float16 activations.
//
// Two Q2_0 weights of one code byte's nibble are each (code - 1) * d, code in 0..3: of their two inputs (a, b)
// they make one of 16 sums, (c & 3 - 1) a + (c >> 2 - 1) b for the nibble c. The table holds those sums for
// every pair of inputs of a token, float16, (tokens, cols / 2, 16). A row's product is then two table reads a
// code byte:
//
//   q2_table_kernel    one thread a (token, input pair): the 16 sums in float32, rounded once to float16; from x,
//                      or from silu(gate) * up (sigmoid in float32 with expf, nothing rounded before the sums).
//   q2_lookup_kernel   a workgroup a (pair, block of rows): the pair's token's table into LDS (copied, or built
//                      there from gate and up: the same code as q2_table_kernel, so the same bits), then P lanes a
//                      row (P = per_row), lane `part` taking runs part, part + P, ...: a run's eight code bytes
//                      add (float(lo) + float(hi)) to a float32 s in order, the run adds d * s to the lane's sum
//                      (one fused multiply-add), and the row's total is lane 0's sum plus lanes 1 .. P - 1's in
//                      that order, rounded once to float16. Gate and up in one launch (two stacks) take the same
//                      path row by row, so they give the bits of two launches.
//
// Tables in LDS are 16 * cols bytes (64 KB for 4096 inputs). The kernels are bound by the table reads (two
// 2-byte LDS reads a code byte), not by HBM.
#include <algorithm>

#include "common.h"

namespace {

constexpr int kLThreads = 256;
constexpr int kLMaxCols = 4096;  // LDS table: cols * 16 bytes

// eight code bytes at 2-byte alignment (gfx950 serves the unaligned 8-byte load as it is)
struct __attribute__((packed, aligned(2))) CodeBytes {
  uint32_t v[2];
};

__device__ __forceinline__ float silu_mul(float g, float u) { return g / (1.0f + expf(-g)) * u; }

// the 16 sums of the input pair (a, b), float16, as eight dwords
__device__ __forceinline__ void pair_sums(float a, float b, uint32_t (&h)[8]) {
#pragma unroll
  for (int c = 0; c < 16; c += 2) {
    const float v0 = (float)((c & 3) - 1) * a + (float)((c >> 2) - 1) * b;
    const float v1 = (float)(((c + 1) & 3) - 1) * a + (float)(((c + 1) >> 2) - 1) * b;
    h[c / 2] = (uint32_t)__builtin_bit_cast(uint16_t, from_f32<f16>(v0)) |
               ((uint32_t)__builtin_bit_cast(uint16_t, from_f32<f16>(v1)) << 16);
  }
}

template <bool GLU>
__device__ __forceinline__ void column_pair(const f16* x, const f16* up, int64_t at, float& a, float& b) {
  if constexpr (GLU) {
    a = silu_mul((float)x[at], (float)up[at]);
    b = silu_mul((float)x[at + 1], (float)up[at + 1]);
  } else {
    a = (float)x[at];
    b = (float)x[at + 1];
  }
}

template <bool GLU>
__global__ __launch_bounds__(kLThreads) void q2_table_kernel(const f16* __restrict__ x, const f16* __restrict__ up,
                                                             int64_t n_pairs, int cols, f16* __restrict__ table) {
  const int64_t i = (int64_t)blockIdx.x * kLThreads + threadIdx.x;  // (token, input pair)
  if (i >= n_pairs) return;
  const int64_t t = i / (cols / 2), g = i % (cols / 2);
  float a, b;
  column_pair<GLU>(x, up, t * cols + 2 * g, a, b);
  uint32_t h[8];
  pair_sums(a, b, h);
  u32x4* dst = reinterpret_cast<u32x4*>(table + i * 16);
  dst[0] = u32x4{h[0], h[1], h[2], h[3]};
  dst[1] = u32x4{h[4], h[5], h[6], h[7]};
}

struct LookupParams {
  const uint8_t* blocks[2];  // one stack, or gate and up
  f16* out[2];
  const uint32_t* idx;
  const f16* table;          // (tokens, cols / 2, 16), or null: built from gate / up
  const f16* gate;
  const f16* up;
  int64_t experts;
  int rows, cols, row_bytes, pairs, share, per_row, rows_per_wg;
};

template <bool TWO, bool GLU>
__global__ __launch_bounds__(kLThreads) void q2_lookup_kernel(LookupParams p) {
  extern __shared__ __attribute__((aligned(16))) f16 tab[];  // cols / 2 * 16
  const int tid = threadIdx.x;
  const int pair = blockIdx.y;
  const int half_cols = p.cols / 2;
  if constexpr (GLU) {  // this pair's table from its gate and up
    for (int g = tid; g < half_cols; g += kLThreads) {
      float a, b;
      column_pair<true>(p.gate, p.up, (int64_t)pair * p.cols + 2 * g, a, b);
      uint32_t h[8];
      pair_sums(a, b, h);
      u32x4* dst = reinterpret_cast<u32x4*>(tab + (int64_t)g * 16);
      dst[0] = u32x4{h[0], h[1], h[2], h[3]};
      dst[1] = u32x4{h[4], h[5], h[6], h[7]};
    }
  } else {  // the pair's token's table, 16-byte copies
    const u32x4* src = reinterpret_cast<const u32x4*>(p.table + (int64_t)(pair / p.share) * half_cols * 16);
    u32x4* dst = reinterpret_cast<u32x4*>(tab);
    for (int i = tid; i < half_cols * 2; i += kLThreads) dst[i] = src[i];
  }
  __syncthreads();

  const uint32_t expert = p.idx[pair];
  const bool bad = expert >= (uint64_t)p.experts;
  const int P = p.per_row;
  const int part = tid % P, rloc = tid / P;
  const int runs = p.cols / 32;
  const int all_rows = TWO ? 2 * p.rows : p.rows;
  const int r0 = blockIdx.x * p.rows_per_wg;
  const int r1 = min(r0 + p.rows_per_wg, all_rows);
  const unsigned char* tb = reinterpret_cast<const unsigned char*>(tab);
  for (int rb = r0; rb < r1; rb += kLThreads / P) {
    const int rr = rb + rloc;
    const bool live = rr < r1;
    int r = live ? rr : r1 - 1;  // past the end: the last row again, not written (the lanes still shuffle)
    const bool second = TWO && r >= p.rows;
    if (second) r -= p.rows;
    const uint8_t* row =
        p.blocks[second ? 1 : 0] + ((int64_t)(bad ? 0u : expert) * p.rows + r) * (int64_t)p.row_bytes;
    float sum = 0.0f;
    for (int n = part; n < runs; n += P) {
      const uint8_t* b = row + (n / 2) * 18;
      const uint8_t* q = b + 2 + 8 * (n % 2);
      const CodeBytes cb = *reinterpret_cast<const CodeBytes*>(q);  // 2-byte aligned, read as it is
      const uint32_t q0 = cb.v[0], q1 = cb.v[1];
      const unsigned char* t = tb + (int64_t)n * 512;  // 256 sums of 2 bytes a run
      float s = 0.0f;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const uint32_t c = ((i < 4 ? q0 : q1) >> (8 * (i & 3))) & 255;
        const float lo = (float)*reinterpret_cast<const f16*>(t + 64 * i + 2 * (c & 15));
        const float hi = (float)*reinterpret_cast<const f16*>(t + 64 * i + 32 + 2 * (c >> 4));
        s += lo + hi;
      }
      const float d = (float)*reinterpret_cast<const f16*>(b);
      sum = __fmaf_rn(d, s, sum);
    }
    float total = sum;
    for (int k = 1; k < P; ++k) total += __shfl_xor(sum, k, P);
    if (live && part == 0) {
      const f16 v = bad ? (f16)__builtin_nanf("") : from_f32<f16>(total);
      p.out[second ? 1 : 0][(int64_t)pair * p.rows + r] = v;
    }
  }
}

int launch_lookup(LookupParams& p, bool two, bool glu, hipStream_t s) {
  const int all_rows = two ? 2 * p.rows : p.rows;
  const int per_pass = kLThreads / p.per_row;
  // rows a workgroup: enough workgroups for the chip, each copying its table for as many rows as that allows
  int passes = (all_rows + per_pass - 1) / per_pass;
  const int64_t want_wgs = 1024;
  const int64_t per_pair_wgs = std::max<int64_t>(1, want_wgs / std::max(1, p.pairs));
  const int passes_per_wg = (int)std::max<int64_t>(1, (passes + per_pair_wgs - 1) / per_pair_wgs);
  p.rows_per_wg = passes_per_wg * per_pass;
  const int gx = (all_rows + p.rows_per_wg - 1) / p.rows_per_wg;
  const size_t smem = (size_t)p.cols * 16;
  dim3 grid(gx, p.pairs);
  if (glu)
    hipLaunchKernelGGL((q2_lookup_kernel<false, true>), grid, dim3(kLThreads), smem, s, p);
  else if (two)
    hipLaunchKernelGGL((q2_lookup_kernel<true, false>), grid, dim3(kLThreads), smem, s, p);
  else
    hipLaunchKernelGGL((q2_lookup_kernel<false, false>), grid, dim3(kLThreads), smem, s, p);
  STRATA_CHECK_LAUNCH();
  return STRATA_OK;
}

int lookup_shape(int64_t experts, int64_t rows, int64_t cols, int64_t pairs, int per_row) {
  if (experts < 1 || rows < 0 || cols < 0 || pairs < 0) return STRATA_ERR_ARG;
  if (cols % 64 || cols > kLMaxCols || rows > (1 << 24) || pairs > 65535) return STRATA_ERR_SHAPE;
  if (per_row < 1 || per_row > 32 || (per_row & (per_row - 1)) || kLThreads % per_row) return STRATA_ERR_ARG;
  return STRATA_OK;
}

}  // namespace

extern "C" {

int strata_q2_lookup_table(const void* x, int64_t tokens, int64_t cols, void* table, void* stream) {
  if (tokens < 0 || cols < 0) return STRATA_ERR_ARG;
  if (tokens == 0 || cols == 0) return STRATA_OK;
  if (!x || !table) return STRATA_ERR_ARG;
  if (cols % 2 || tokens * cols > ((int64_t)1 << 32)) return STRATA_ERR_SHAPE;
  const int64_t n = tokens * (cols / 2);
  hipLaunchKernelGGL((q2_table_kernel<false>), dim3((unsigned)((n + kLThreads - 1) / kLThreads)), dim3(kLThreads), 0,
                     (hipStream_t)stream, (const f16*)x, (const f16*)nullptr, n, (int)cols, (f16*)table);
  STRATA_CHECK_LAUNCH();
  return STRATA_OK;
}

int strata_q2_lookup_table_glu(const void* gate, const void* up, int64_t tokens, int64_t cols, void* table,
                               void* stream) {
  if (tokens < 0 || cols < 0) return STRATA_ERR_ARG;
  if (tokens == 0 || cols == 0) return STRATA_OK;
  if (!gate || !up || !table) return STRATA_ERR_ARG;
  if (cols % 2 || tokens * cols > ((int64_t)1 << 32)) return STRATA_ERR_SHAPE;
  const int64_t n = tokens * (cols / 2);
  hipLaunchKernelGGL((q2_table_kernel<true>), dim3((unsigned)((n + kLThreads - 1) / kLThreads)), dim3(kLThreads), 0,
                     (hipStream_t)stream, (const f16*)gate, (const f16*)up, n, (int)cols, (f16*)table);
  STRATA_CHECK_LAUNCH();
  return STRATA_OK;
}

int strata_q2_lookup_matvec(const void* blocks, const void* blocks_b, int64_t experts, int64_t rows, int64_t cols,
                            const uint32_t* idx, int64_t pairs, const void* table, int64_t share, int per_row,
                            void* out, void* out_b, void* stream) {
  int rc = lookup_shape(experts, rows, cols, pairs, per_row);
  if (rc) return rc;
  if (pairs == 0 || rows == 0) return STRATA_OK;
  if (!blocks || !idx || !table || !out || (blocks_b != nullptr) != (out_b != nullptr)) return STRATA_ERR_ARG;
  if (share < 1 || pairs % share) return STRATA_ERR_ARG;
  LookupParams p = {};
  p.blocks[0] = (const uint8_t*)blocks;
  p.blocks[1] = (const uint8_t*)blocks_b;
  p.out[0] = (f16*)out;
  p.out[1] = (f16*)out_b;
  p.idx = idx;
  p.table = (const f16*)table;
  p.experts = experts;
  p.rows = (int)rows;
  p.cols = (int)cols;
  p.row_bytes = (int)(cols / 64 * 18);
  p.pairs = (int)pairs;
  p.share = (int)share;
  p.per_row = per_row;
  return launch_lookup(p, blocks_b != nullptr, false, (hipStream_t)stream);
}

int strata_q2_lookup_down_glu(const void* blocks, int64_t experts, int64_t rows, int64_t cols, const uint32_t* idx,
                              int64_t pairs, const void* gate, const void* up, int per_row, void* out, void* stream) {
  int rc = lookup_shape(experts, rows, cols, pairs, per_row);
  if (rc) return rc;
  if (pairs == 0 || rows == 0) return STRATA_OK;
  if (!blocks || !idx || !gate || !up || !out) return STRATA_ERR_ARG;
  LookupParams p = {};
  p.blocks[0] = (const uint8_t*)blocks;
  p.out[0] = (f16*)out;
  p.idx = idx;
  p.gate = (const f16*)gate;
  p.up = (const f16*)up;
  p.experts = experts;
  p.rows = (int)rows;
  p.cols = (int)cols;
  p.row_bytes = (int)(cols / 64 * 18);
  p.pairs = (int)pairs;
  p.share = 1;
  p.per_row = per_row;
  return launch_lookup(p, false, true, (hipStream_t)stream);
}

}  // extern "C"
