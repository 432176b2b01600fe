// Either side of the expert path: the router's product, its top-k choice with the softmax of the chosen logits,
// and the combine of the experts' outputs with the shared expert (strata_mlx/fused.py:357-497).
//
//   router_matvec  out[t, r] = W[r, :] . x[t, :], W float16 (rows x cols), x float16 / float32, sums float32.
//                  A wave a row: 64 lanes read the row with 16-byte loads (coalesced), v_dot2 against each
//                  token's activations, a DPP reduction; HBM-bound (2 MB for 256 x 4096).
//   top_k          a wave a row of logits: the k largest, ties to the lower index (the order a stable sort
//                  gives), in descending order; and the softmax of the chosen logits in float32.
//   moe_combine    out = (half)(sum_k y_k * w_k) + (half)((half)sigmoid(g) * s), the experts added in the order
//                  of strata_mlx/fused.py:448-466 (eight partial sums, expert j into sum j % 8, each product
//                  rounded before it is added, the sums in order), every half operation rounded once.
//   router_route   router_matvec and top_k in one launch at up to 8 tokens: the last workgroup to finish its
//                  rows takes the choice, and rounds the rows past the experts' (a shared expert's gate) to half.
#include <type_traits>
#include <math.h>

#include <algorithm>

#include "common.h"
#include "topk.h"

namespace {

using strata_topk::top_k_row;

constexpr int kWaves = 4;  // waves a workgroup

template <int CTRL>
__device__ __forceinline__ float dpp_mov(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xF, 0xF, false));
}

__device__ __forceinline__ float wave_sum(float v) {
  v += dpp_mov<0xB1>(v);   // lanes ^ 1
  v += dpp_mov<0x4E>(v);   // lanes ^ 2
  v += dpp_mov<0x141>(v);  // mirror within 8
  v += dpp_mov<0x140>(v);  // mirror within 16
  v += __shfl_xor(v, 16);
  v += __shfl_xor(v, 32);
  return v;
}

typedef _Float16 h2_t __attribute__((ext_vector_type(2)));

// Row `row` of W against every token (at most 8): the wave's sums, the same in every lane. A lane's pieces of the
// row (16 bytes each, 512 columns apart) are asked for eight at a time, and a token's pieces of x the same way,
// before any is used: one wait for memory where a piece at a time waited eight times (the router of 256 x 4096
// at one token: 7.4 us a launch). Each sum adds the pieces in column order, as one piece at a time did.
template <typename XT>
__device__ __forceinline__ void router_row(const f16* __restrict__ w, int row, int cols, const XT* __restrict__ x,
                                           int tokens, int lane, float (&sums)[8]) {
  constexpr int kPieces = 8;
  const f16* wr = w + (int64_t)row * cols;
  float acc[8];
#pragma unroll
  for (int t = 0; t < 8; ++t) acc[t] = 0.0f;
  for (int c0 = lane * 8; c0 < cols; c0 += 512 * kPieces) {
    u32x4 wv[kPieces];
#pragma unroll
    for (int p = 0; p < kPieces; ++p)
      if (c0 + 512 * p < cols) wv[p] = *reinterpret_cast<const u32x4*>(wr + c0 + 512 * p);
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      if (t < tokens) {
        if constexpr (sizeof(XT) == 2) {
          u32x4 xv[kPieces];
#pragma unroll
          for (int p = 0; p < kPieces; ++p)
            if (c0 + 512 * p < cols) xv[p] = *reinterpret_cast<const u32x4*>(x + (int64_t)t * cols + c0 + 512 * p);
#pragma unroll
          for (int p = 0; p < kPieces; ++p) {
            if (c0 + 512 * p < cols) {
#pragma unroll
              for (int i = 0; i < 4; ++i) {
                // elements copied out first: a bit cast of a vector element lvalue reads element 0 whatever the index
                const uint32_t wi = wv[p][i], xi = xv[p][i];
                acc[t] = __builtin_amdgcn_fdot2(__builtin_bit_cast(h2_t, wi), __builtin_bit_cast(h2_t, xi), acc[t],
                                                false);
              }
            }
          }
        } else {
#pragma unroll
          for (int p = 0; p < kPieces; ++p) {
            const int c = c0 + 512 * p;
            if (c < cols) {
#pragma unroll
              for (int i = 0; i < 4; ++i) {
                const uint32_t wi = wv[p][i];
                const h2_t pw = __builtin_bit_cast(h2_t, wi);
                acc[t] += (float)pw[0] * x[(int64_t)t * cols + c + 2 * i] + (float)pw[1] * x[(int64_t)t * cols + c + 2 * i + 1];
              }
            }
          }
        }
      }
    }
  }
#pragma unroll
  for (int t = 0; t < 8; ++t) sums[t] = t < tokens ? wave_sum(acc[t]) : 0.0f;
}

// One wave a row, all tokens (at most 8 a launch; the host splits longer inputs).
template <typename XT>
__global__ __launch_bounds__(256) void router_matvec_kernel(const f16* __restrict__ w, int rows, int cols,
                                                            const XT* __restrict__ x, int tokens,
                                                            float* __restrict__ out) {
  const int lane = threadIdx.x % 64;
  const int row = blockIdx.x * kWaves + threadIdx.x / 64;
  if (row >= rows) return;
  float sums[8];
  router_row<XT>(w, row, cols, x, tokens, lane, sums);
#pragma unroll
  for (int t = 0; t < 8; ++t)
    if (t < tokens && lane == 0) out[(int64_t)t * rows + row] = sums[t];
}

// One wave a row of n <= 64 NV logits (NV a lane); k <= 64.
template <int NV>
__global__ __launch_bounds__(256) void top_k_kernel(const float* __restrict__ logits, int rows, int n, int k,
                                                    uint32_t* __restrict__ idx, float* __restrict__ weights) {
  const int lane = threadIdx.x % 64;
  const int row = blockIdx.x * kWaves + threadIdx.x / 64;
  if (row >= rows) return;
  const float* lr = logits + (int64_t)row * n;
  float v[NV];
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int j = i * 64 + lane;
    v[i] = j < n ? lr[j] : -INFINITY;
  }
  top_k_row<NV>(v, n, k, lane, idx + (int64_t)row * k, weights != nullptr ? weights + (int64_t)row * k : nullptr);
}

// A float at p read where every XCD's stores of it land (sc1, as an agent-scope load), not waited for: the caller
// waits (vmcnt) before it uses the value, so that several of these are in flight at once.
__device__ __forceinline__ float load_agent(const float* p) {
  float r;
  asm volatile("global_load_dword %0, %1, off sc1" : "=v"(r) : "v"(p) : "memory");
  return r;
}

// router_matvec and top_k in one launch (at most 8 tokens). Every workgroup writes its rows' sums (logits, tokens x
// rows) by agent-scope stores (sc1: to the point where every XCD reads them), waits until they are done, then adds
// one to `count`; the workgroup that brings it to the grid's size takes, for each token, the top k of its first
// `experts` logits and their softmax (a wave a token), rounds the rows past them to half into `extra` (tokens x
// (rows - experts), or null), and sets `count` back to zero for the next launch. Nothing waits on another
// workgroup: the others end once their rows are out. (Release and acquire fences in place of the waits wrote back
// and invalidated the L2 in every workgroup: 17.8 us a launch, against 7.4 + 6.8 us for the two launches.)
constexpr int kRouteWaves = 4;  // waves a workgroup of router_route_kernel (16 measured no faster)

template <typename XT, int NV>
__global__ __launch_bounds__(64 * kRouteWaves) void router_route_kernel(const f16* __restrict__ w, int rows, int cols,
                                                           const XT* __restrict__ x, int tokens, float* logits,
                                                           int experts, int k, uint32_t* __restrict__ idx,
                                                           float* __restrict__ weights, f16* __restrict__ extra,
                                                           uint32_t* count) {
  const int lane = threadIdx.x % 64, wave = threadIdx.x / 64;
  const int row = blockIdx.x * kRouteWaves + wave;
  if (row < rows) {
    float sums[8];
    router_row<XT>(w, row, cols, x, tokens, lane, sums);
#pragma unroll
    for (int t = 0; t < 8; ++t)
      if (t < tokens && lane == 0)
        __hip_atomic_store(logits + (int64_t)t * rows + row, sums[t], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __shared__ uint32_t last;
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this wave's stores are done
  __syncthreads();                                   // and every wave's
  if (threadIdx.x == 0)
    last = __hip_atomic_fetch_add(count, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == gridDim.x - 1u;
  __syncthreads();
  if (last == 0u) return;
  asm volatile("" ::: "memory");  // the logits are read after the count
  const int nx = rows - experts;
  // the rows past the experts' (tokens x nx values, two a thread a pass), then each token's choice (a wave a token);
  // all of a thread's loads of a pass in flight together
  constexpr int kExtra = 2;  // extra values a thread per pass
  for (int i0 = 0; extra != nullptr && i0 < tokens * nx; i0 += 64 * kRouteWaves * kExtra) {
    float e[kExtra];
#pragma unroll
    for (int q = 0; q < kExtra; ++q) {
      const int i = min(i0 + q * 64 * kRouteWaves + (int)threadIdx.x, tokens * nx - 1);
      e[q] = load_agent(logits + (int64_t)(i / nx) * rows + experts + i % nx);
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
#pragma unroll
    for (int q = 0; q < kExtra; ++q) asm volatile("" : "+v"(e[q]));  // used only after the wait
#pragma unroll
    for (int q = 0; q < kExtra; ++q) {
      const int i = i0 + q * 64 * kRouteWaves + (int)threadIdx.x;
      if (i < tokens * nx) extra[i] = from_f32<f16>(e[q]);
    }
  }
  for (int t = wave; t < tokens; t += kRouteWaves) {
    float v[NV];
#pragma unroll
    for (int i = 0; i < NV; ++i) v[i] = load_agent(logits + (int64_t)t * rows + min(i * 64 + lane, experts - 1));
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
#pragma unroll
    for (int i = 0; i < NV; ++i) asm volatile("" : "+v"(v[i]));  // used only after the wait
#pragma unroll
    for (int i = 0; i < NV; ++i)
      if (i * 64 + lane >= experts) v[i] = -INFINITY;
    top_k_row<NV>(v, experts, k, lane, idx + (int64_t)t * k, weights != nullptr ? weights + (int64_t)t * k : nullptr);
  }
  if (threadIdx.x == 0) __hip_atomic_store(count, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// One thread an output element.
__global__ __launch_bounds__(256) void moe_combine_kernel(const f16* __restrict__ y, const float* __restrict__ w,
                                                          const f16* __restrict__ g, const f16* __restrict__ s,
                                                          int k, int d, f16* __restrict__ out) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  const int t = blockIdx.y;
  if (i >= d) return;
  float acc = 0.0f;
  for (int j = 0; j < 8 && j < k; ++j) {
    float part = 0.0f;
    for (int q = j; q < k; q += 8)
      part = __fadd_rn(__fmul_rn((float)y[((int64_t)t * k + q) * d + i], w[(int64_t)t * k + q]), part);
    acc = j == 0 ? part : __fadd_rn(part, acc);
  }
  const f16 routed = from_f32<f16>(acc);
  const f16 gate = from_f32<f16>(1.0f / (1.0f + expf(-(float)g[t])));
  const f16 shared = from_f32<f16>((float)gate * (float)s[(int64_t)t * d + i]);  // exact product, one rounding
  out[(int64_t)t * d + i] = routed + shared;                                      // a float16 add: one rounding
}

}  // namespace

extern "C" {

int strata_router_matvec(const void* w, int64_t rows, int64_t cols, const void* x, int64_t tokens, int x_dtype,
                         float* out, void* stream) {
  if (rows < 0 || cols < 0 || tokens < 0) return STRATA_ERR_ARG;
  if (rows == 0 || tokens == 0) return STRATA_OK;
  if (!w || !x || !out) return STRATA_ERR_ARG;
  if (cols % 8 || rows > INT32_MAX / 2 || cols > (1 << 24)) return STRATA_ERR_SHAPE;
  if (x_dtype != DT_F16 && x_dtype != DT_F32) return STRATA_ERR_DTYPE;
  const int grid = (int)((rows + kWaves - 1) / kWaves);
  hipStream_t s = (hipStream_t)stream;
  for (int64_t t0 = 0; t0 < tokens; t0 += 8) {
    const int nt = (int)std::min<int64_t>(8, tokens - t0);
    if (x_dtype == DT_F16)
      hipLaunchKernelGGL(router_matvec_kernel<f16>, dim3(grid), dim3(256), 0, s, (const f16*)w, (int)rows,
                         (int)cols, (const f16*)x + t0 * cols, nt, out + t0 * rows);
    else
      hipLaunchKernelGGL(router_matvec_kernel<float>, dim3(grid), dim3(256), 0, s, (const f16*)w, (int)rows,
                         (int)cols, (const float*)x + t0 * cols, nt, out + t0 * rows);
    STRATA_CHECK_LAUNCH();
  }
  return STRATA_OK;
}

int strata_top_k(const float* logits, int64_t rows, int64_t n, int64_t k, uint32_t* idx, float* weights,
                 void* stream) {
  if (rows < 0 || n < 0 || k < 0) return STRATA_ERR_ARG;
  if (rows == 0 || k == 0) return STRATA_OK;
  if (!logits || !idx) return STRATA_ERR_ARG;
  if (n > 2048 || k > 64 || k > n || rows > INT32_MAX / 2) return STRATA_ERR_SHAPE;
  const int grid = (int)((rows + kWaves - 1) / kWaves);
  // the logits a lane holds: the row's length over 64, rounded up to a power of two
  auto launch = [&](auto nv) {
    hipLaunchKernelGGL(top_k_kernel<decltype(nv)::value>, dim3(grid), dim3(256), 0, (hipStream_t)stream, logits,
                       (int)rows, (int)n, (int)k, idx, weights);
  };
  if (n <= 64) launch(std::integral_constant<int, 1>{});
  else if (n <= 128) launch(std::integral_constant<int, 2>{});
  else if (n <= 256) launch(std::integral_constant<int, 4>{});
  else if (n <= 512) launch(std::integral_constant<int, 8>{});
  else if (n <= 1024) launch(std::integral_constant<int, 16>{});
  else launch(std::integral_constant<int, 32>{});
  STRATA_CHECK_LAUNCH();
  return STRATA_OK;
}

int strata_router_route(const void* w, int64_t rows, int64_t cols, const void* x, int64_t tokens, int x_dtype,
                        float* logits, int64_t experts, int64_t k, uint32_t* idx, float* weights, void* extra,
                        uint32_t* count, void* stream) {
  if (rows < 0 || cols < 0 || tokens < 0 || experts < 0 || k < 0) return STRATA_ERR_ARG;
  if (tokens == 0) return STRATA_OK;
  if (!w || !x || !logits || !idx || !count || k == 0 || experts == 0) return STRATA_ERR_ARG;
  if (cols % 8 || cols > (1 << 24) || experts > rows || rows > INT32_MAX / 2) return STRATA_ERR_SHAPE;
  if (tokens > 8 || experts > 2048 || k > 64 || k > experts) return STRATA_ERR_SHAPE;
  if (x_dtype != DT_F16 && x_dtype != DT_F32) return STRATA_ERR_DTYPE;
  const int grid = (int)((rows + kRouteWaves - 1) / kRouteWaves);
  auto launch = [&](auto xt, auto nv) {
    typedef decltype(xt) XT;
    hipLaunchKernelGGL((router_route_kernel<XT, decltype(nv)::value>), dim3(grid), dim3(64 * kRouteWaves), 0,
                       (hipStream_t)stream,
                       (const f16*)w, (int)rows, (int)cols, (const XT*)x, (int)tokens, logits, (int)experts, (int)k,
                       idx, weights, (f16*)extra, count);
  };
  auto by_n = [&](auto xt) {
    if (experts <= 64) launch(xt, std::integral_constant<int, 1>{});
    else if (experts <= 128) launch(xt, std::integral_constant<int, 2>{});
    else if (experts <= 256) launch(xt, std::integral_constant<int, 4>{});
    else if (experts <= 512) launch(xt, std::integral_constant<int, 8>{});
    else if (experts <= 1024) launch(xt, std::integral_constant<int, 16>{});
    else launch(xt, std::integral_constant<int, 32>{});
  };
  if (x_dtype == DT_F16)
    by_n(f16{});
  else
    by_n(0.0f);
  STRATA_CHECK_LAUNCH();
  return STRATA_OK;
}

int strata_moe_combine(const void* y, const float* w, const void* g, const void* s, int64_t rows, int64_t k,
                       int64_t d, int dtype, void* out, void* stream) {
  if (rows < 0 || k < 0 || d < 0) return STRATA_ERR_ARG;
  if (rows == 0 || d == 0) return STRATA_OK;
  if (!y || !w || !g || !s || !out || k == 0) return STRATA_ERR_ARG;
  if (dtype != DT_F16) return STRATA_ERR_DTYPE;
  if (rows > 65535 || d > INT32_MAX / 2) return STRATA_ERR_SHAPE;
  hipLaunchKernelGGL(moe_combine_kernel, dim3((int)((d + 255) / 256), (int)rows), dim3(256), 0, (hipStream_t)stream,
                     (const f16*)y, w, (const f16*)g, (const f16*)s, (int)k, (int)d, (f16*)out);
  STRATA_CHECK_LAUNCH();
  return STRATA_OK;
}

}  // extern "C"
