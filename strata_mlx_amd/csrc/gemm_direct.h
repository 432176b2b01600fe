// The prompt kernel for IQ3_S, IQ3_XXS and Q2_0 rows of whole 256-weight blocks, 16-bit activations.
//
// c[s, :] = W[e(s)] . a[s, :] over tiles of 16 slots, each tile one expert's (strata_mlx/blocks.py:583-654).
// A workgroup (kGWaves waves) takes 16 output rows a wave of one expert and its tiles within an aligned window of
// kDTiles tiles; it is the workgroup at the group's first tile that works, the others of the column exit at once.
// A K step is 256 columns (one IQ3 block, four Q2_0 blocks, of every row), eight runs of 32, one MFMA each:
// v_mfma_f32_16x16x32_f16, a (16 slots x 32) x w (32 x 16 rows). Lane (n, g) of a wave gives the MFMA row n's
// columns 8g .. 8g + 7 of the run, which are groups 2g and 2g + 1 of the run. A wave stages its 16 rows' bytes
// of the step in its own LDS slab (coalesced 16-byte loads, a step ahead); each lane reads back exactly its
// fields (the two index or code bytes, and the run's shared sign, scale and high-bit fields) and decodes them in
// registers into exact float16 integers (codebook entry with its sign). The product times the row's run scale
// is added to the float32 sums, so nothing is rounded. The group's activations for a step go to LDS (bfloat16
// converted to float16 on the way), shared by the workgroup's waves. An expert's weights are read and decoded
// once per window of kDTiles tiles it has tiles in: two tiles a window keeps the kernel under 90 VGPRs (five or
// six waves a SIMD), which is worth more than decoding the weights of experts with three or more tiles again.
#pragma once
#include "direct_impl.h"
#include "gemm_impl.h"

namespace strata_gemm {

constexpr int kGWaves = 8;                   // waves a workgroup
constexpr int kGThreads = 64 * kGWaves;
constexpr int kDRows = 16 * kGWaves;         // output rows a workgroup
constexpr int kDStep = 256;                  // columns a K step
constexpr int kDPitch = kDStep + 8;          // LDS pitch of a slot's activations (float16), against bank conflicts
constexpr int kDTiles = 2;                   // tiles a group
constexpr int kDRuns = kDStep / 32;          // runs of a row a step: one MFMA each

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

// A K step of a row as the kernel stages it: the step's bytes (one IQ3 block, four Q2_0 blocks) in 16-byte chunks,
// the last one ending at the step's end.
template <int KIND>
struct StepBytes {
  static constexpr int bytes = KIND == K_IQ3_S ? 110 : KIND == K_IQ3_XXS ? 98 : 72;
  static constexpr int chunks = (bytes + 15) / 16;
  static constexpr int pitch = 16 * chunks;  // a row's bytes in the slab (28 or 20 dwords: the 16 rows' fields
                                             // fall in different banks)
  __device__ static int offset(int c) { return min(16 * c, bytes - 16); }
};

template <typename T>
__device__ __forceinline__ T lds_load(const uint8_t* p) {
  typedef const __attribute__((address_space(3))) strata_mv::Unaligned<T> L;
  return ((L*)(const __attribute__((address_space(3))) uint8_t*)p)->v;
}
template <typename T>
__device__ __forceinline__ void lds_store(uint8_t* p, T v) {
  typedef __attribute__((address_space(3))) strata_mv::Unaligned<T> L;
  ((L*)(__attribute__((address_space(3))) uint8_t*)p)->v = v;
}

// Lane slice g of a step's bytes b (in LDS): each run's two index (code) bytes of groups 2g and 2g + 1, and the
// run's shared fields.
template <int KIND>
__device__ __forceinline__ void read_slice(const uint8_t* b, int g, StepSlice<KIND>& f) {
  if constexpr (KIND == K_IQ3_S) {  // d @0, qs[64] @2, qh[8] @66, signs[32] @74, scales[4] @106
    f.d = lds_load<uint16_t>(b);
#pragma unroll
    for (int q = 0; q < kDRuns; ++q) f.qs[q] = lds_load<uint16_t>(b + 2 + 8 * q + 2 * g);
    f.qh = lds_load<u32x2>(b + 66);
    f.sg[0] = lds_load<u32x4>(b + 74);
    f.sg[1] = lds_load<u32x4>(b + 90);
    f.sc = lds_load<uint32_t>(b + 106);
  } else if constexpr (KIND == K_IQ3_XXS) {  // d @0, qs[64] @2, aux[8] (u32) @66
    f.d = lds_load<uint16_t>(b);
#pragma unroll
    for (int q = 0; q < kDRuns; ++q) f.qs[q] = lds_load<uint16_t>(b + 2 + 8 * q + 2 * g);
    f.aux[0] = lds_load<u32x4>(b + 66);
    f.aux[1] = lds_load<u32x4>(b + 82);
  } else {  // Q2_0, four blocks of 18 bytes (d @0, qs[16] @2); run q: block q / 2, code bytes 8 (q % 2) on
#pragma unroll
    for (int j = 0; j < kDRuns / 2; ++j) f.d[j] = lds_load<uint16_t>(b + 18 * j);
#pragma unroll
    for (int q = 0; q < kDRuns; ++q) f.qs[q] = lds_load<uint16_t>(b + 18 * (q / 2) + 2 + 8 * (q % 2) + 2 * g);
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
// one a thread a tile), as they are in memory: they are converted when they go to LDS, a step later, so that
// nothing waits for them before then.
template <typename AT>
__device__ __forceinline__ void load_step_acts(const AT* a, const GemmParams& p, int t0, int nt, int k, int tid,
                                               u32x4 (&av)[kDTiles]) {
  static_assert(kGThreads == 16 * (kDStep / 8), "one 16-byte chunk of a tile's step a thread");
  const int slot = tid / (kDStep / 8), col = (tid % (kDStep / 8)) * 8;
#pragma unroll
  for (int i = 0; i < kDTiles; ++i)
    if (i < nt) av[i] = *reinterpret_cast<const u32x4*>(a + ((int64_t)(t0 + i) * 16 + slot) * p.cols + k * kDStep + col);
}

// The chunks to LDS as float16 (bfloat16 converted: exact in float16's range).
template <typename AT>
__device__ __forceinline__ void store_step_acts(f16* a_lds, int nt, int tid, const u32x4 (&av)[kDTiles]) {
#pragma unroll
  for (int i = 0; i < kDTiles; ++i) {
    if (i < nt) {
      u32x4 o = av[i];
      if constexpr (!std::is_same<AT, f16>::value) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const float lo = __uint_as_float(av[i][q] << 16), hi = __uint_as_float(av[i][q] & 0xffff0000u);
          o[q] = (uint32_t)__builtin_bit_cast(uint16_t, (f16)lo) |
                 ((uint32_t)__builtin_bit_cast(uint16_t, (f16)hi) << 16);
        }
      }
      *reinterpret_cast<u32x4*>(a_lds + (i * 16 + tid / 32) * kDPitch + (tid % 32) * 8) = o;
    }
  }
}

// The K loop of a group of up to NT tiles (nt of them). A wave stages its 16 rows' bytes of a step in its own LDS
// slab: two 16-byte loads a lane (chunk L of the 16 rows' chunks: row L / chunks), loaded a step ahead, written to
// the slab when the step comes, then read back as the lanes' slices. One wave writes and reads its slab, so no
// barrier guards it (a wave's LDS operations are done in order). The activations of step k + 1 are loaded while
// step k is multiplied.
template <int KIND, typename AT, int NT>
__device__ __forceinline__ void group_product(const GemmParams& p, const strata_mv::DirectTables<KIND>& tab,
                                              f16* a_lds, uint8_t* slab, const uint8_t* mat, int n0w, int t0,
                                              int row, int tid, int nt) {
  using SB = StepBytes<KIND>;
  const int lane = tid % 64, n = lane % 16, g = lane / 16;
  const AT* a = reinterpret_cast<const AT*>(p.a);
  const int nsteps = p.cols / kDStep;

  // the lane's two chunks: rows and offsets (lanes past the 16 rows' chunks load the last again, write nothing)
  constexpr int kChunks = 16 * SB::chunks;
  static_assert(kChunks <= 128, "two chunks a lane");
  const uint8_t* src[2];
  int dst[2];
  bool put[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int L = min(lane + 64 * h, kChunks - 1);
    const int r = L / SB::chunks, c = L % SB::chunks;
    src[h] = mat + (int64_t)min(n0w + r, p.rows - 1) * p.row_bytes + SB::offset(c);
    dst[h] = r * SB::pitch + SB::offset(c);
    put[h] = lane + 64 * h < kChunks;
  }
  u32x4 raw[2][2];  // the ring: step k's chunks, step k + 1's in flight
#pragma unroll
  for (int h = 0; h < 2; ++h) raw[0][h] = strata_mv::load_unaligned<u32x4>(src[h]);
  u32x4 av[kDTiles];
  load_step_acts<AT>(a, p, t0, nt, 0, tid, av);

  f32x4 acc[NT];
#pragma unroll
  for (int i = 0; i < NT; ++i) acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};

  for (int kb = 0; kb < nsteps; kb += 2) {
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const int k = kb + s;
      if (k < nsteps) {
        // step k + 1's chunks (past the last step the last again: unconditional loads, which the waits for
        // earlier loads can count on)
        const int64_t next = (int64_t)min(k + 1, nsteps - 1) * SB::bytes;
#pragma unroll
        for (int h = 0; h < 2; ++h) raw[(s + 1) % 2][h] = strata_mv::load_unaligned<u32x4>(src[h] + next);
        __syncthreads();  // every wave's reads of the last step's activations are done (and the tables written)
        store_step_acts<AT>(a_lds, nt, tid, av);
        if (k + 1 < nsteps) load_step_acts<AT>(a, p, t0, nt, k + 1, tid, av);
#pragma unroll
        for (int h = 0; h < 2; ++h)
          if (put[h]) lds_store<u32x4>(slab + dst[h], raw[s][h]);
        StepSlice<KIND> f;
        read_slice<KIND>(slab + n * SB::pitch, g, f);
        __syncthreads();
#pragma unroll
        for (int q = 0; q < kDRuns; ++q) {
          uint32_t w[4];
          const float sc = decode_slice<KIND>(f, q, g, w, tab);
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
  __shared__ __attribute__((aligned(16))) uint8_t slabs[kGWaves * 16 * StepBytes<KIND>::pitch];

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
  const uint8_t* mat = p.blocks + (int64_t)e * p.mat_bytes;
  {
    strata_mv::TableFetch<KIND> tf;
    strata_mv::fetch_tables<KIND, kGThreads>(tf, tid);
    strata_mv::store_tables<KIND, kGThreads>(tab, tf, tid);  // read after the K loop's first barrier
  }
  nt = __builtin_amdgcn_readfirstlane(nt);
  group_product<KIND, AT, kDTiles>(p, tab, a_lds, slabs + wave * 16 * StepBytes<KIND>::pitch, mat, n0 + wave * 16,
                                    t0, row, tid, nt);
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
