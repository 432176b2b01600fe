// The prompt kernel for IQ3_S, IQ3_XXS and Q2_0 rows of whole 256-weight blocks, 16-bit activations.
//
// c[s, :] = W[e(s)] . a[s, :] over tiles of 16 slots, each tile one expert's (strata_mlx/blocks.py:583-654).
// A workgroup (4 waves) takes 64 output rows of one expert and its tiles within an aligned window of four tiles;
// it is the workgroup at the group's first tile that works, the others of the column exit at once. For each K step of
// 256 columns (one IQ3 block, four Q2_0 blocks, of every row):
//   - each thread loads the fields of one run pair (64 weights) of one row straight into registers and decodes
//     them into LDS as float16 integers, exact (codebook entry with its sign), and the two runs' scales as
//     float32: nothing is rounded;
//   - the group's activations for the step go to LDS too (bfloat16 converted to float16 as they load);
//   - each wave multiplies its 16 rows by every tile, one run (32 columns) at a time on v_mfma_f32_16x16x32_f16:
//     a (16 slots x 32) x w (32 x 16 rows), and adds the product times each row's run scale to its float32 sums.
// An expert's weights are read and decoded once per window of four tiles it has tiles in.
#pragma once
#include "direct_impl.h"
#include "gemm_impl.h"

namespace strata_gemm {

constexpr int kDRows = 64;                 // output rows a workgroup
constexpr int kDStep = 256;                // columns a K step
constexpr int kDPitch = kDStep + 8;        // LDS pitch of a row / slot (float16), against bank conflicts
constexpr int kDTiles = 4;                 // tiles a group
constexpr int kDRuns = kDStep / 32;        // runs of a row a step

constexpr int kDAhead = 4;                 // K steps the weights' loads run ahead

// The fields of run pair dj of K step k of a row (64 weights).
template <int KIND>
__device__ __forceinline__ void load_step_fields(const uint8_t* row, int k, int dj, strata_mv::RunPair<KIND>& f) {
  strata_mv::load_fields<KIND>(row, 0, strata_mv::lane_offsets<KIND>(k * (kDStep / 64) + dj), f);
}

// This thread's share of K step k's activations of the group (16-byte chunks of 16 slots x 256 columns a tile),
// as float16.
template <typename AT>
__device__ __forceinline__ void load_step_acts(const AT* a, const GemmParams& p, int t0, int nt, int k, int tid,
                                               u32x4 (&av)[kDTiles * 2]) {
#pragma unroll
  for (int i = 0; i < kDTiles; ++i) {
    if (i < nt) {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int c = tid + h * kThreads;
        const int slot = c / (kDStep / 8), col = (c % (kDStep / 8)) * 8;
        const AT* src = a + ((int64_t)(t0 + i) * 16 + slot) * p.cols + k * kDStep + col;
        if constexpr (std::is_same<AT, f16>::value) {
          av[2 * i + h] = *reinterpret_cast<const u32x4*>(src);
        } else {
          const u32x4 raw = *reinterpret_cast<const u32x4*>(src);  // 8 bfloat16
          u32x4 o;
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const float lo = __uint_as_float(raw[q] << 16), hi = __uint_as_float(raw[q] & 0xffff0000u);
            o[q] = (uint32_t)__builtin_bit_cast(uint16_t, (f16)lo) |
                   ((uint32_t)__builtin_bit_cast(uint16_t, (f16)hi) << 16);
          }
          av[2 * i + h] = o;
        }
      }
    }
  }
}

template <int KIND, typename AT>
__global__ __launch_bounds__(kThreads, 2) void direct_gemm_kernel(GemmParams p) {
  __shared__ strata_mv::DirectTables<KIND> tab;
  __shared__ __attribute__((aligned(16))) f16 w_lds[kDRows * kDPitch];
  __shared__ float s_lds[kDRows * kDRuns];
  __shared__ __attribute__((aligned(16))) f16 a_lds[kDTiles * 16 * kDPitch];

  const int tid = threadIdx.x, lane = tid % 64;
  const int wave = __builtin_amdgcn_readfirstlane(tid / 64);
  const int n0 = blockIdx.x * kDRows;
  const int t0 = blockIdx.y;

  // the group: the tiles of expert e in t0's aligned window of kDTiles tiles, from t0 on, when t0 is the first
  // of them (a window's first tile, or an expert's); deciding it reads at most kDTiles ids, all at once
  const uint32_t e = p.tile_expert[t0];
  if (e >= (uint64_t)p.experts) return;
  if (t0 % kDTiles != 0 && p.tile_expert[t0 - 1] == e) return;
  const int wend = min((t0 / kDTiles + 1) * kDTiles, p.n_tiles);
  int nt = 1;
#pragma unroll
  for (int i = 1; i < kDTiles; ++i)
    if (t0 + i < wend && nt == i && p.tile_expert[t0 + i] == e) nt = i + 1;

  {
    strata_mv::TableFetch<KIND> tf;
    strata_mv::fetch_tables<KIND>(tf, tid);
    strata_mv::store_tables<KIND>(tab, tf, tid);
  }
  const uint8_t* mat = p.blocks + (int64_t)e * p.mat_bytes;
  const AT* a = reinterpret_cast<const AT*>(p.a);
  // decode share: row dr, run pair dj of the step
  const int dr = tid / 4, dj = tid % 4;
  const int drow = min(n0 + dr, p.rows - 1);
  const uint8_t* wrow = mat + (int64_t)drow * p.row_bytes;

  f32x4 acc[kDTiles];
#pragma unroll
  for (int i = 0; i < kDTiles; ++i) acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};

  // Loads run ahead of the work: the weights' fields kDAhead steps, the activations one step (issued before the
  // fields, so that waiting for them is not waiting for the later fields).
  const int nsteps = p.cols / kDStep;
  strata_mv::RunPair<KIND> f[kDAhead];
#pragma unroll
  for (int s = 0; s < kDAhead; ++s)
    if (s < nsteps) load_step_fields<KIND>(wrow, s, dj, f[s]);
  u32x4 av[kDTiles * 2];
  load_step_acts<AT>(a, p, t0, nt, 0, tid, av);

  for (int kb = 0; kb < nsteps; kb += kDAhead) {
#pragma unroll
    for (int s = 0; s < kDAhead; ++s) {
      const int k = kb + s;
      if (k < nsteps) {
        strata_mv::opaque(f[s]);
        __syncthreads();  // the last step's LDS is read
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          uint32_t w[16];
          const float scale = strata_mv::decode_pair<KIND>(f[s], h, w, tab);
          u32x4* dst = reinterpret_cast<u32x4*>(w_lds + dr * kDPitch + 64 * dj + 32 * h);
#pragma unroll
          for (int v = 0; v < 4; ++v) dst[v] = u32x4{w[4 * v], w[4 * v + 1], w[4 * v + 2], w[4 * v + 3]};
          s_lds[dr * kDRuns + 2 * dj + h] = scale;
        }
#pragma unroll
        for (int i = 0; i < kDTiles; ++i) {
          if (i < nt) {
#pragma unroll
            for (int h = 0; h < 2; ++h) {
              const int c = tid + h * kThreads;
              const int slot = c / (kDStep / 8), col = (c % (kDStep / 8)) * 8;
              *reinterpret_cast<u32x4*>(a_lds + (i * 16 + slot) * kDPitch + col) = av[2 * i + h];
            }
          }
        }
        if (k + 1 < nsteps) load_step_acts<AT>(a, p, t0, nt, k + 1, tid, av);
        if (k + kDAhead < nsteps) load_step_fields<KIND>(wrow, k + kDAhead, dj, f[s]);
        __syncthreads();
        // wave: rows 16 wave + n, n = lane % 16; k slice 8 (lane / 16) of each run
        const int n = lane % 16, g = lane / 16;
        const f16* wr = w_lds + (wave * 16 + n) * kDPitch + 8 * g;
#pragma unroll
        for (int q = 0; q < kDRuns; ++q) {
          const f16x8 bv = *reinterpret_cast<const f16x8*>(wr + 32 * q);
          const float sc = s_lds[(wave * 16 + n) * kDRuns + q];
#pragma unroll
          for (int i = 0; i < kDTiles; ++i) {
            if (i < nt) {
              const f16x8 av8 = *reinterpret_cast<const f16x8*>(a_lds + (i * 16 + n) * kDPitch + 32 * q + 8 * g);
              const f32x4 d = __builtin_amdgcn_mfma_f32_16x16x32_f16(av8, bv, f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
#pragma unroll
              for (int j = 0; j < 4; ++j) acc[i][j] += d[j] * sc;
            }
          }
        }
      }
    }
  }
  // lane holds slots 4 g + j of each tile for row n
  const int row = n0 + wave * 16 + lane % 16;
  if (row < p.rows) {
    for (int i = 0; i < nt; ++i) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int64_t s = (int64_t)(t0 + i) * 16 + 4 * (lane / 16) + j;
        p.c[s * p.rows + row] = acc[i][j];
      }
    }
  }
}

template <int KIND>
int launch_direct_gemm(GemmParams& p, int a_dtype, hipStream_t s) {
  dim3 grid((p.rows + kDRows - 1) / kDRows, p.n_tiles);
  if (a_dtype == DT_F16)
    hipLaunchKernelGGL((direct_gemm_kernel<KIND, f16>), grid, dim3(kThreads), 0, s, p);
  else
    hipLaunchKernelGGL((direct_gemm_kernel<KIND, bf16_t>), grid, dim3(kThreads), 0, s, p);
  STRATA_CHECK_LAUNCH();
  return STRATA_OK;
}

}  // namespace strata_gemm
