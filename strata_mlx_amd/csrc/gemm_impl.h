// The prompt kernel: a grouped dequant-matmul over tiles of slots, each tile one expert's, on CDNA4 MFMA.
//
// c[s, :] = W[e(s)] . a[s, :] where slot s is in a tile of 16 whose expert is tile_expert[s / 16]
// (strata_mlx/blocks.py:583-654). A workgroup (4 waves) takes 64 rows of the output and a group of up to
// four consecutive tiles; consecutive tiles of one expert share every weight it decodes. For each K step
// of 64 columns it decodes the 64 x 64 weights into LDS once (as float16 for 16-bit activations, exact
// float32 for float32 ones), and each wave multiplies its 16 rows against every tile of the group:
//   float16 v_mfma_f32_16x16x32_f16: a (16 slots x 32 cols) x w (32 cols x 16 rows), float32 sums; bfloat16
//           activations come as rows scaled into float16 by a power of two (a_max: each row's largest
//           magnitude), and the sums are scaled back by it
//   float32 v_mfma_f32_16x16x4_f32, exact weights.
#pragma once
#include <type_traits>

#include "decode.h"

namespace strata_gemm {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;
constexpr int kRowsBlock = 64;   // output rows per workgroup (4 waves x 16)
constexpr int kGroupTiles = 4;   // tiles per workgroup
constexpr int kKStep = 64;       // columns decoded per step

struct GemmParams {
  const uint8_t* blocks;
  const void* a;
  const uint32_t* a_max;  // float16 rows scaled by a power of two: each row's largest magnitude, or null
  const uint32_t* tile_expert;
  float* c;
  int64_t experts, mat_bytes;
  int rows, cols, row_bytes, n_tiles;
};

__device__ __forceinline__ f16x8 load_a8(const f16* src) { return *reinterpret_cast<const f16x8*>(src); }

template <int KIND, typename AT, int GT>
__global__ __launch_bounds__(kThreads) void tile_gemm_kernel(GemmParams p) {
  constexpr bool kF32 = std::is_same<AT, float>::value;
  using WT = typename std::conditional<kF32, float, f16>::type;
  constexpr int kPitch = kKStep + (kF32 ? 4 : 8);  // LDS row pitch, padded against bank conflicts
  __shared__ StrataTables tab;
  __shared__ __attribute__((aligned(16))) WT w_lds[kRowsBlock * kPitch];

  const int tid = threadIdx.x, wave = tid / 64, lane = tid % 64;
  const int n0 = blockIdx.x * kRowsBlock;
  const int t_begin = blockIdx.y * GT;
  const int t_end = min(t_begin + GT, p.n_tiles);
  const AT* a = reinterpret_cast<const AT*>(p.a);
  strata_load_tables<KIND>(tab);

  int t = t_begin;
  while (t < t_end) {
    const uint32_t e = p.tile_expert[t];
    int t1 = t + 1;
    while (t1 < t_end && p.tile_expert[t1] == e) ++t1;
    if (e >= (uint64_t)p.experts) {  // a tile nothing fills: left out
      t = t1;
      continue;
    }
    const uint8_t* mat = p.blocks + (int64_t)e * p.mat_bytes;
    const int ntile = t1 - t;
    f32x4 acc[GT];
#pragma unroll
    for (int i = 0; i < GT; ++i) acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};

    for (int k0 = 0; k0 < p.cols; k0 += kKStep) {
      __syncthreads();  // the tables are in; the last step's weights are read
      for (int u = tid; u < kRowsBlock * (kKStep / 32); u += kThreads) {
        const int r = u / (kKStep / 32), part = u % (kKStep / 32);
        WT* dst = w_lds + r * kPitch + 32 * part;
        if (n0 + r < p.rows) {
          float w[32];
          strata_unpack32<KIND>(mat + (int64_t)(n0 + r) * p.row_bytes, (uint32_t)(k0 / 32 + part), w, tab);
#pragma unroll
          for (int j = 0; j < 32; ++j) dst[j] = (WT)w[j];
        } else {
#pragma unroll
          for (int j = 0; j < 32; ++j) dst[j] = (WT)0.0f;
        }
      }
      __syncthreads();
      const WT* wrow = w_lds + (wave * 16 + lane % 16) * kPitch;
#pragma unroll
      for (int i = 0; i < GT; ++i) {
        if (i < ntile) {
          const AT* arow = a + ((int64_t)(t + i) * 16 + lane % 16) * p.cols + k0;
          if constexpr (kF32) {
#pragma unroll
            for (int kk = 0; kk < kKStep; kk += 4)
              acc[i] = __builtin_amdgcn_mfma_f32_16x16x4f32(arow[kk + lane / 16], wrow[kk + lane / 16], acc[i], 0, 0, 0);
          } else {
#pragma unroll
            for (int kk = 0; kk < kKStep; kk += 32) {
              const f16x8 av = load_a8(reinterpret_cast<const f16*>(arow + kk + 8 * (lane / 16)));
              const f16x8 bv = *reinterpret_cast<const f16x8*>(wrow + kk + 8 * (lane / 16));
              acc[i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, bv, acc[i], 0, 0, 0);
            }
          }
        }
      }
    }
    const int n = n0 + wave * 16 + lane % 16;
    if (n < p.rows) {
#pragma unroll
      for (int i = 0; i < GT; ++i) {
        if (i < ntile) {
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const int64_t s = (int64_t)(t + i) * 16 + 4 * (lane / 16) + j;
            p.c[s * p.rows + n] = p.a_max ? __builtin_ldexpf(acc[i][j], row_exponent(p.a_max[s])) : acc[i][j];
          }
        }
      }
    }
    t = t1;
  }
}

template <int KIND, int GT>
int launch_gemm_group(GemmParams& p, int a_dtype, hipStream_t s) {
  dim3 grid((p.rows + kRowsBlock - 1) / kRowsBlock, (p.n_tiles + GT - 1) / GT);
  if (grid.y > 65535) return STRATA_ERR_SHAPE;
  if (a_dtype == DT_F16)
    hipLaunchKernelGGL((tile_gemm_kernel<KIND, f16, GT>), grid, dim3(kThreads), 0, s, p);
  else if (a_dtype == DT_F32)
    hipLaunchKernelGGL((tile_gemm_kernel<KIND, float, GT>), grid, dim3(kThreads), 0, s, p);
  else
    return STRATA_ERR_DTYPE;
  STRATA_CHECK_LAUNCH();
  return STRATA_OK;
}

// A stack of one matrix (a dense layer's chunk of tokens, every tile the same expert) decodes each weight tile
// once for kDenseTiles tiles; routed tiles, mostly one or two an expert, go kGroupTiles to a workgroup.
constexpr int kDenseTiles = 16;
template <int KIND>
int launch_gemm_kind(GemmParams& p, int a_dtype, hipStream_t s) {
  if (p.experts == 1 && p.n_tiles >= kDenseTiles) return launch_gemm_group<KIND, kDenseTiles>(p, a_dtype, s);
  return launch_gemm_group<KIND, kGroupTiles>(p, a_dtype, s);
}

}  // namespace strata_gemm
