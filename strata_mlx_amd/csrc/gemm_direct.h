// The prompt kernel for IQ3_S, IQ3_XXS and Q2_0 rows of whole 256-weight blocks, 16-bit activations.
//
// c[s, :] = W[e(s)] . a[s, :] over tiles of 16 slots, each tile one expert's (strata_mlx/blocks.py:583-654).
// A workgroup (kGWaves waves) takes 16 output rows a wave of one expert and its tiles within an aligned window of
// four tiles; it is the workgroup at the group's first tile that works, the others of the column exit at once.
// A K step is 256 columns (one IQ3 block, four Q2_0 blocks, of every row), eight runs of 32, one MFMA each:
// v_mfma_f32_16x16x32_f16, a (16 slots x 32) x w (32 x 16 rows). Lane (n, g) of a wave gives the MFMA row n's
// columns 8g .. 8g + 7 of the run, which are groups 2g and 2g + 1 of the run: it loads exactly their fields (the
// two index or code bytes, and the run's shared sign, scale and high-bit fields) and decodes them in registers
// into exact float16 integers (codebook entry with its sign). The product times the row's run scale is added to
// the float32 sums, so nothing is rounded. The weights never pass through LDS; the group's activations for a
// step do (bfloat16 converted to float16 as they load), shared by the workgroup's waves. An expert's weights
// are read and decoded once per window of four tiles it has tiles in.
#pragma once
#include "direct_impl.h"
#include "gemm_impl.h"

namespace strata_gemm {

constexpr int kGWaves = 8;                   // waves a workgroup
constexpr int kGThreads = 64 * kGWaves;
constexpr int kDRows = 16 * kGWaves;         // output rows a workgroup
constexpr int kDStep = 256;                  // columns a K step
constexpr int kDPitch = kDStep + 8;          // LDS pitch of a slot's activations (float16), against bank conflicts
constexpr int kDTiles = 4;                   // tiles a group
constexpr int kDRuns = kDStep / 32;          // runs of a row a step: one MFMA each
constexpr int kDRing = 2;                    // K steps of fields held: the one decoded and one loading

// What lane slice g of one row holds of a K step: each run's two index (code) bytes for groups 2g and 2g + 1,
// and the fields the run's groups share.
template <int KIND>
struct StepSlice;
template <>
struct StepSlice<K_IQ3_S> {
  uint32_t qs[kDRuns];  // two index bytes a run
  u32x2 qh;             // the eight high-bit bytes (byte q: the ninth index bits of run q's groups)
  u32x4 sg[2];          // the 32 sign bytes (byte 4q + g: groups 2g, 2g + 1 of run q)
  uint32_t sc;          // the four scale bytes (nibble q: run q)
  uint32_t d;
};
template <>
struct StepSlice<K_IQ3_XXS> {
  uint32_t qs[kDRuns];
  u32x4 aux[2];  // the runs' scale and sign words
  uint32_t d;
};
template <>
struct StepSlice<K_Q2_0> {
  uint32_t qs[kDRuns];     // two code bytes a run
  uint32_t d[kDRuns / 2];  // a block's d (two runs a block)
};

template <int KIND>
__device__ __forceinline__ void load_slice(const uint8_t* row, int k, int g, StepSlice<KIND>& f) {
  using strata_mv::load_unaligned;
  if constexpr (KIND == K_IQ3_S) {  // d @0, qs[64] @2, qh[8] @66, signs[32] @74, scales[4] @106
    const uint8_t* b = row + k * 110;
    f.d = load_unaligned<uint16_t>(b);
#pragma unroll
    for (int q = 0; q < kDRuns; ++q) f.qs[q] = load_unaligned<uint16_t>(b + 2 + 8 * q + 2 * g);
    f.qh = load_unaligned<u32x2>(b + 66);
    f.sg[0] = load_unaligned<u32x4>(b + 74);
    f.sg[1] = load_unaligned<u32x4>(b + 90);
    f.sc = load_unaligned<uint32_t>(b + 106);
  } else if constexpr (KIND == K_IQ3_XXS) {  // d @0, qs[64] @2, aux[8] (u32) @66
    const uint8_t* b = row + k * 98;
    f.d = load_unaligned<uint16_t>(b);
#pragma unroll
    for (int q = 0; q < kDRuns; ++q) f.qs[q] = load_unaligned<uint16_t>(b + 2 + 8 * q + 2 * g);
    f.aux[0] = load_unaligned<u32x4>(b + 66);
    f.aux[1] = load_unaligned<u32x4>(b + 82);
  } else {  // Q2_0, four blocks of 18 bytes (d @0, qs[16] @2); run q: block q / 2, code bytes 8 (q % 2) on
    const uint8_t* b = row + k * 72;
#pragma unroll
    for (int j = 0; j < kDRuns / 2; ++j) f.d[j] = load_unaligned<uint16_t>(b + 18 * j);
#pragma unroll
    for (int q = 0; q < kDRuns; ++q) f.qs[q] = load_unaligned<uint16_t>(b + 18 * (q / 2) + 2 + 8 * (q % 2) + 2 * g);
  }
}

// The compiler no longer knows the fields' values: their decode cannot move above this point (nor its waits
// for the loads).
template <int KIND>
__device__ __forceinline__ void opaque_slice(StepSlice<KIND>& f) {
#pragma unroll
  for (int q = 0; q < kDRuns; ++q) asm volatile("" : "+v"(f.qs[q]));
  if constexpr (KIND == K_IQ3_S) {
    asm volatile("" : "+v"(f.qh), "+v"(f.sg[0]), "+v"(f.sg[1]), "+v"(f.sc), "+v"(f.d));
  } else if constexpr (KIND == K_IQ3_XXS) {
    asm volatile("" : "+v"(f.aux[0]), "+v"(f.aux[1]), "+v"(f.d));
  } else {
#pragma unroll
    for (int j = 0; j < kDRuns / 2; ++j) asm volatile("" : "+v"(f.d[j]));
  }
}

// Run q of the slice: groups 2g and 2g + 1 as four packed float16 pairs of integers into w, exact; returns the
// run's scale (float32, exact).
template <int KIND>
__device__ __forceinline__ float decode_slice(const StepSlice<KIND>& f, int q, int g, uint32_t (&w)[4],
                                              const strata_mv::DirectTables<KIND>& t) {
  using strata_mv::half_bits;
  u32x2 g0, g1, m0, m1;
  float scale;
  if constexpr (KIND == K_IQ3_S) {  // strata_mlx/blocks.py:89-102
    const uint32_t hb = (f.qh[q / 4] >> (8 * (q % 4) + 2 * g)) & 3;
    const uint32_t sg = (f.sg[q / 4][q % 4] >> (8 * g)) & 255;
    g0 = t.grid[(f.qs[q] & 255) | ((hb & 1) << 8)];
    g1 = t.grid[((f.qs[q] >> 8) & 255) | ((hb >> 1) << 8)];
    m0 = t.sign4[sg & 15];
    m1 = t.sign4[sg >> 4];
    scale = half_bits(f.d) * (float)(1 + 2 * ((f.sc >> (4 * q)) & 15));
  } else if constexpr (KIND == K_IQ3_XXS) {  // strata_mlx/blocks.py:103-116
    const uint32_t a = f.aux[q / 4][q % 4];
    const uint32_t s7 = (a >> (7 * g)) & 127;
    const uint32_t s8 = s7 | ((__builtin_popcount(s7) & 1u) << 7);  // ksigns: the parity in bit 7
    g0 = t.grid[f.qs[q] & 255];
    g1 = t.grid[(f.qs[q] >> 8) & 255];
    m0 = t.sign4[s8 & 15];
    m1 = t.sign4[s8 >> 4];
    scale = half_bits(f.d) * (0.5f + (float)(a >> 28)) * 0.5f;
  } else {  // Q2_0, strata_mlx/blocks.py:58-68: a code byte's four (c - 1)
    g0 = t.q2[f.qs[q] & 255];
    g1 = t.q2[(f.qs[q] >> 8) & 255];
    m0 = m1 = u32x2{0u, 0u};
    scale = half_bits(f.d[q / 2]);
  }
  w[0] = g0[0] ^ m0[0];
  w[1] = g0[1] ^ m0[1];
  w[2] = g1[0] ^ m1[0];
  w[3] = g1[1] ^ m1[1];
  return scale;
}

// This thread's share of K step k's activations of the group (16-byte chunks of 16 slots x 256 columns a tile:
// one a thread a tile), as float16.
template <typename AT>
__device__ __forceinline__ void load_step_acts(const AT* a, const GemmParams& p, int t0, int nt, int k, int tid,
                                               u32x4 (&av)[kDTiles]) {
  static_assert(kGThreads == 16 * (kDStep / 8), "one 16-byte chunk of a tile's step a thread");
  const int slot = tid / (kDStep / 8), col = (tid % (kDStep / 8)) * 8;
#pragma unroll
  for (int i = 0; i < kDTiles; ++i) {
    if (i < nt) {
      const AT* src = a + ((int64_t)(t0 + i) * 16 + slot) * p.cols + k * kDStep + col;
      if constexpr (std::is_same<AT, f16>::value) {
        av[i] = *reinterpret_cast<const u32x4*>(src);
      } else {
        const u32x4 raw = *reinterpret_cast<const u32x4*>(src);  // 8 bfloat16
        u32x4 o;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const float lo = __uint_as_float(raw[q] << 16), hi = __uint_as_float(raw[q] & 0xffff0000u);
          o[q] = (uint32_t)__builtin_bit_cast(uint16_t, (f16)lo) |
                 ((uint32_t)__builtin_bit_cast(uint16_t, (f16)hi) << 16);
        }
        av[i] = o;
      }
    }
  }
}

// The K loop of a group of NT tiles (a template parameter: the loop is straight-line code, which the compiler
// interleaves: decode of one run with the MFMAs and sums of the last). Fields of step k + kDRing - 1 are loaded
// while step k is decoded; the activations of step k + 1 while step k is multiplied.
template <int KIND, typename AT, int NT>
__device__ __forceinline__ void group_product(const GemmParams& p, const strata_mv::DirectTables<KIND>& tab,
                                              f16* a_lds, const uint8_t* wrow, int t0, int row, int tid, int nt) {
  const int lane = tid % 64, n = lane % 16, g = lane / 16;
  const AT* a = reinterpret_cast<const AT*>(p.a);
  const int nsteps = p.cols / kDStep;

  StepSlice<KIND> f[kDRing];
#pragma unroll
  for (int s = 0; s < kDRing - 1; ++s)
    if (s < nsteps) load_slice<KIND>(wrow, s, g, f[s]);
  u32x4 av[kDTiles];
  load_step_acts<AT>(a, p, t0, nt, 0, tid, av);

  f32x4 acc[NT];
#pragma unroll
  for (int i = 0; i < NT; ++i) acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};

  for (int kb = 0; kb < nsteps; kb += kDRing) {
#pragma unroll
    for (int s = 0; s < kDRing; ++s) {
      const int k = kb + s;
      if (k < nsteps) {
        // fields of step k + kDRing - 1 go to the ring slot step k - 1 used
        if (k + kDRing - 1 < nsteps) load_slice<KIND>(wrow, k + kDRing - 1, g, f[(s + kDRing - 1) % kDRing]);
        __syncthreads();  // every wave's reads of the last step's activations are done (and the tables written)
#pragma unroll
        for (int i = 0; i < NT; ++i)
          if (i < nt) *reinterpret_cast<u32x4*>(a_lds + (i * 16 + tid / 32) * kDPitch + (tid % 32) * 8) = av[i];
        if (k + 1 < nsteps) load_step_acts<AT>(a, p, t0, nt, k + 1, tid, av);
        opaque_slice<KIND>(f[s]);
        __syncthreads();
#pragma unroll
        for (int q = 0; q < kDRuns; ++q) {
          uint32_t w[4];
          const float sc = decode_slice<KIND>(f[s], q, g, w, tab);
          const f16x8 bv = __builtin_bit_cast(f16x8, u32x4{w[0], w[1], w[2], w[3]});
#pragma unroll
          for (int i = 0; i < NT; ++i) {
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
  if (row < p.rows) {
    for (int i = 0; i < nt; ++i) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int64_t s = (int64_t)(t0 + i) * 16 + 4 * g + j;
        p.c[s * p.rows + row] = acc[i][j];
      }
    }
  }
}

template <int KIND, typename AT>
__global__ __launch_bounds__(kGThreads, 4) void direct_gemm_kernel(GemmParams p) {
  __shared__ strata_mv::DirectTables<KIND> tab;
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

  // lane (n, g): row n of the wave's 16, columns 8g .. 8g + 7 of each run
  const int row = n0 + wave * 16 + lane % 16;
  const uint8_t* wrow = p.blocks + (int64_t)e * p.mat_bytes + (int64_t)min(row, p.rows - 1) * p.row_bytes;
  {
    strata_mv::TableFetch<KIND> tf;
    strata_mv::fetch_tables<KIND, kGThreads>(tf, tid);
    strata_mv::store_tables<KIND, kGThreads>(tab, tf, tid);  // read after the K loop's first barrier
  }
  static_assert(kDTiles == 4, "one K loop for each group size");
  nt = __builtin_amdgcn_readfirstlane(nt);
  group_product<KIND, AT, 4>(p, tab, a_lds, wrow, t0, row, tid, nt);
}

template <int KIND>
int launch_direct_gemm(GemmParams& p, int a_dtype, hipStream_t s) {
  dim3 grid((p.rows + kDRows - 1) / kDRows, p.n_tiles);
  if (a_dtype == DT_F16)
    hipLaunchKernelGGL((direct_gemm_kernel<KIND, f16>), grid, dim3(kGThreads), 0, s, p);
  else
    hipLaunchKernelGGL((direct_gemm_kernel<KIND, bf16_t>), grid, dim3(kGThreads), 0, s, p);
  STRATA_CHECK_LAUNCH();
  return STRATA_OK;
}

}  // namespace strata_gemm
