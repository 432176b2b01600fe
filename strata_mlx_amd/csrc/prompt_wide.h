// The prompt kernels' wide form: the full chunks of 16 tiles of the experts with many tiles, each expert's rows
// decoded once for all 16 tiles in a step's LDS shared by a workgroup's eight waves (strata_mlx/blocks.py:583-694).
// A run of one expert's tiles of length L is split: its first 16 * floor(L / 16) tiles go to this kernel in chunks
// of 16, the rest (the tail) to the chunked form (prompt_impl.h, with PromptParams.skip_full), which takes it in
// chunks of up to three from the tail's first tile. The two launches write disjoint slots.
//
// One workgroup a CU (8 waves, 144 KB of LDS), persistent. A work item is a chunk and a block of 128 weight rows
// (the SwiGLU form: 64 rows of gate and the same 64 of up). For each step of 256 columns every wave decodes one
// group of 16 of the item's rows into LDS, and then every wave multiplies its two tiles of the chunk (tiles w and
// w + 8 of wave w) against all 128 rows: the decode of a step, which bounds the chunked form, is shared by 16 tiles
// in place of 3. On chunks this full it runs at 1.4 times the chunked form (a layer of 64 experts of 16 tiles each:
// 516 against 359 TFLOPS); on every chunk of a Zipf routing it ran slower (243 against 360): in short chunks the
// waves without a tile wait at every step's barrier.
//
// The weights reach the MFMAs as the chunked form gives them, exact float16 integers with the run's scale folded
// in (decode_folded4), and what a row's step shares (IQ3_S d, IQ3_XXS d / 4) is not folded in. One float32 sum a
// slot and row runs through every step, kept divided by the row's step scale in force: before step k's products
// the sums are multiplied by s / d_k (s the scale of the last step whose d was not zero), which the decoding lane
// writes to LDS beside the weights, and after the last step by the last such scale. (Q2_0's weights carry their
// scale.)
//
// Double-buffered decoded steps (2 x 64 KB): a wave decodes step k + 1 into one buffer, then multiplies step k
// from the other, then meets the others at the step's one barrier, after which both buffers change roles. A wave's
// own fields are loaded two steps ahead, and the activations of its tiles (16 slots each, read by row index
// straight into MFMA operand registers) one step ahead, each register asked for again once step k's MFMAs have
// read it.
//
// Work is dealt without device state: every workgroup first lists the full chunks in LDS from the tiles' experts
// (up to kWideMaxTiles tiles), then takes items in turn: item i is chunk i / R, row block i % R (R row blocks), on
// workgroup i % G of G (a multiple of 8). Workgroup w runs on XCD w % 8; with R a multiple of 8 (a 1536- or
// 4096-row layer) row block r of every chunk runs on XCD r % 8, so the chunks of one expert read the same rows at
// about the same time from one L2.
#pragma once
#include "prompt_impl.h"

namespace strata_prompt {

constexpr int kWideWaves = 8;                         // waves a workgroup
constexpr int kWidePerCU = 1;                         // workgroups a CU
constexpr int kWideWavesSimd = 2;                     // waves a SIMD the kernel is built for
constexpr int kWideThreads = 64 * kWideWaves;
constexpr int kWideGroups = kWideWaves;               // groups of 16 weight rows an item
constexpr int kGroupsWave = kWideGroups / kWideWaves;  // groups a wave decodes
constexpr int kWideTilesWave = 2;                     // tiles a wave multiplies at most
constexpr int kWideChunk = kWideWaves * kWideTilesWave;  // tiles a chunk
static_assert(kWideChunk == kFullChunk, "the chunked form's tails start where the full chunks end");
constexpr int kWideMaxTiles = 5120;                   // tiles the plan takes (its chunk list is in LDS)
constexpr int kWideBuf = kWideGroups * 8 * 64;        // 16-byte pieces of a decoded step: [group][MFMA][lane]

template <int MODE>
constexpr int wide_out_rows() {  // output rows an item
  return MODE == PM_GLU ? 16 * kWideGroups / 2 : 16 * kWideGroups;
}

// The workgroup's exclusive prefix of v over its threads in order (sum, or max with -1 for none), and the total.
template <bool MAX>
__device__ __forceinline__ int wide_scan(int v, int* scratch, int tid, int& total) {
  const int lane = tid & 63, wave = tid >> 6;
  const int none = MAX ? -1 : 0;
  int incl = v;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int o = __shfl_up(incl, d);
    if (lane >= d) incl = MAX ? max(incl, o) : incl + o;
  }
  int excl = __shfl_up(incl, 1);
  if (lane == 0) excl = none;
  if (lane == 63) scratch[wave] = incl;
  __syncthreads();
  int before = none;
  total = none;
#pragma unroll
  for (int w = 0; w < kWideWaves; ++w) {
    const int s = scratch[w];
    if (w < wave) before = MAX ? max(before, s) : before + s;
    total = MAX ? max(total, s) : total + s;
  }
  __syncthreads();  // the scratch is free again
  return MAX ? max(before, excl) : before + excl;
}

// The full chunks' first tiles, in order, into chunks; returns their number. A chunk starts at every tile whose
// offset from its run's first tile (a run: consecutive tiles of one expert, wherever they lie: an expert may have
// several) is a multiple of kWideChunk and whose run goes on for kWideChunk tiles from it; tiles naming no expert
// make none. Thread t looks at tiles 20 t .. 20 t + 19.
__device__ __forceinline__ int wide_plan(const PromptParams& p, uint16_t* chunks, int* scratch, int tid) {
  constexpr int kPer = kWideMaxTiles / kWideThreads;
  static_assert(kPer * kWideThreads == kWideMaxTiles, "whole tiles a thread");
  const int n = p.n_tiles, i0 = tid * kPer;
  uint32_t tv[kPer];
#pragma unroll
  for (int k = 0; k < kPer; ++k) tv[k] = i0 + k < n ? p.tile_expert[i0 + k] : 0u;
  const uint32_t prev = i0 > 0 && i0 - 1 < n ? p.tile_expert[i0 - 1] : 0u;
  int last = -1;  // the last run start among the thread's tiles
  {
    uint32_t pv = prev;
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
      const int i = i0 + k;
      if (i < n) {
        if (i == 0 || tv[k] != pv) last = i;
        pv = tv[k];
      }
    }
  }
  int ignored;
  const int start_in = wide_scan<true>(last, scratch, tid, ignored);  // the run start in force before i0
  auto starts = [&](auto&& at) {
    uint32_t pv = prev;
    int r = start_in;
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
      const int i = i0 + k;
      if (i < n) {
        if (i == 0 || tv[k] != pv) r = i;
        pv = tv[k];
        if ((uint64_t)tv[k] < (uint64_t)p.experts && (i - r) % kWideChunk == 0 && i + kWideChunk - 1 < n) {
          bool full = true;  // every tile of the block names the run's expert (a run: contiguous tiles of one)
          for (int j = 1; j < kWideChunk && full; ++j) full = p.tile_expert[i + j] == tv[k];
          if (full) at(i);
        }
      }
    }
  };
  int cnt = 0;
  starts([&](int) { ++cnt; });
  int total;
  int base = wide_scan<false>(cnt, scratch, tid, total);
  starts([&](int i) { chunks[base++] = (uint16_t)i; });
  __syncthreads();
  return total;
}

// A step's weights of this wave's group: 16 rows, lane (n, g) row n's run pair g (runs 2 g, 2 g + 1: columns
// 64 g .. 64 g + 63), into the buffer as MFMA operands, exact. MFMA s of a step takes columns 32 s .. 32 s + 31, lane
// (n, q) of it columns 32 s + 8 q .. + 7, so that its activations are 64 contiguous bytes of each slot's row: the
// decoding lane's weights 8 q .. 8 q + 7 of run h go to MFMA 2 g + h, lane 16 q + n. With a step scale, lane (n, 0)
// writes row n's ratio s / d_k to ratio[n] (see the top of this file; s, the lane's scale in force, moves to d_k
// unless d_k is zero).
template <int KIND>
__device__ __forceinline__ void wide_decode(const RunPair<KIND>& f, int g, const DirectTables<KIND>& tab,
                                            u32x4* dst, float* ratio, float& s, int lane) {
  const int n = lane & 15;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      uint32_t w[4];
      decode_folded4<KIND>(f, h, g, q, w, tab);
      dst[(2 * g + h) * 64 + 16 * q + n] = u32x4{w[0], w[1], w[2], w[3]};
    }
  }
  if constexpr (has_step_scale<KIND>()) {
    const float dk = step_scale<KIND>(f);
    const float r = dk != 0.0f ? s / dk : 1.0f;
    s = dk != 0.0f ? dk : s;
    if (g == 0) ratio[lane] = r;
  }
}

// One item: chunk tiles t0 .. t0 + nt - 1 of expert e, row block rb; this wave's NTW tiles (t0 + wave + 4 i). Every
// wave runs the same steps and barriers whatever its NTW.
template <int KIND, int MODE, typename OT, int NTW>
__device__ __forceinline__ void wide_item(const PromptParams& p, const DirectTables<KIND>& tab, u32x4* wdec,
                                          float* ratio, float* last, uint32_t e, int t0, int rb, int wave, int lane) {
  const int n = lane & 15, g = lane >> 4;
  constexpr bool kGlu = MODE == PM_GLU;
  // this wave's groups of rows, wave + kWideWaves j: SwiGLU form, the first half of the groups gate rows, the second
  // the same rows of up
  constexpr int kHalf = kWideGroups / 2;
  const uint8_t* mat[kGroupsWave];
  uint32_t off[kGroupsWave];
#pragma unroll
  for (int j = 0; j < kGroupsWave; ++j) {
    const int gi = wave + kWideWaves * j;
    const int grow = kGlu ? rb * 16 * kHalf + 16 * (gi % kHalf) + n : rb * 16 * kWideGroups + 16 * gi + n;
    mat[j] = (kGlu && gi >= kHalf ? p.blocks[1] : p.blocks[0]) + (int64_t)e * p.mat_bytes;
    off[j] = (uint32_t)min(grow, p.rows - 1) * (uint32_t)p.row_bytes;  // past the last row: the last
  }
  const LaneOffsets<KIND> o = strata_mv::lane_offsets<KIND>(g);
  const int nsteps = p.cols / kStep;
  const uint32_t step_bytes = (uint32_t)(p.row_bytes / nsteps);

  const f16* arow[NTW > 0 ? NTW : 1];
#pragma unroll
  for (int i = 0; i < NTW; ++i) {
    const int slot = (t0 + wave + kWideWaves * i) * 16 + n;
    const uint32_t r = p.a_row ? p.a_row[slot] : (uint32_t)slot;
    arow[i] = p.a + (int64_t)r * p.cols;
  }

  RunPair<KIND> f[2][kGroupsWave];  // f[s % 2][j]: step s's fields of group j
  float s[kGroupsWave];              // the decoding lane's rows: the step scale in force
  // ratio: [step parity][group][row]; last: [group][row], the scale in force after the last step
  auto decode = [&](int k, int slot) {
#pragma unroll
    for (int j = 0; j < kGroupsWave; ++j) {
      const int gi = wave + kWideWaves * j;
      wide_decode<KIND>(f[slot][j], g, tab, wdec + (k & 1) * kWideBuf + gi * 8 * 64,
                        ratio + (k & 1) * (16 * kWideGroups) + gi * 16, s[j], lane);
      if (k + 1 == nsteps && g == 0) last[gi * 16 + n] = s[j];
    }
  };
  auto fields = [&](int k, int slot) {
#pragma unroll
    for (int j = 0; j < kGroupsWave; ++j)
      strata_mv::load_fields<KIND>(mat[j], off[j] + (uint32_t)k * step_bytes, o, f[slot][j]);
  };
#pragma unroll
  for (int j = 0; j < kGroupsWave; ++j) s[j] = 1.0f;
  fields(0, 0);
  fields(nsteps > 1 ? 1 : 0, 1);
  decode(0, 0);
  if (nsteps > 2) fields(2, 0);
  lds_barrier();

  f32x4 acc[kWideGroups][NTW > 0 ? NTW : 1];
#pragma unroll
  for (int gi = 0; gi < kWideGroups; ++gi)
#pragma unroll
    for (int i = 0; i < NTW; ++i) acc[gi][i] = f32x4{0.f, 0.f, 0.f, 0.f};
  // the activations of the wave's tiles, [MFMA s][tile]: slot n's columns 32 s + 8 g .. + 7 of the step; step k + 1's
  // into each register as soon as step k's MFMAs have read it
  f16x8 a[8][NTW > 0 ? NTW : 1];
  auto load_a = [&](int k, int s) {
#pragma unroll
    for (int i = 0; i < NTW; ++i) a[s][i] = *reinterpret_cast<const f16x8*>(arow[i] + k * kStep + 32 * s + 8 * g);
  };
#pragma unroll
  for (int s = 0; s < 8; ++s) load_a(0, s);

  for (int kb = 0; kb < nsteps; kb += 2) {
#pragma unroll
    for (int sp = 0; sp < 2; ++sp) {
      const int k = kb + sp;
      if (k < nsteps) {
        if (k + 1 < nsteps) {  // step k + 1 into the other buffer, then its fields' slot takes step k + 3's
          decode(k + 1, sp ^ 1);
          if (k + 3 < nsteps) fields(k + 3, sp ^ 1);
        }
        if constexpr (NTW > 0 && has_step_scale<KIND>()) {  // the sums into step k's scale
#pragma unroll
          for (int gi = 0; gi < kWideGroups; ++gi) {
            const float r = ratio[(k & 1) * (16 * kWideGroups) + gi * 16 + n];
#pragma unroll
            for (int i = 0; i < NTW; ++i) acc[gi][i] *= r;
          }
        }
        if constexpr (NTW > 0) {
          const u32x4* buf = wdec + (k & 1) * kWideBuf;
#pragma unroll
          for (int s = 0; s < 8; ++s) {
#pragma unroll
            for (int gi = 0; gi < kWideGroups; ++gi) {
              const f16x8 b = __builtin_bit_cast(f16x8, buf[(gi * 8 + s) * 64 + lane]);
#pragma unroll
              for (int i = 0; i < NTW; ++i)
                acc[gi][i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[s][i], b, acc[gi][i], 0, 0, 0);
            }
            if (k + 1 < nsteps) load_a(k + 1, s);
          }
        }
        if (NTW > 0 && has_step_scale<KIND>() && k + 1 == nsteps) {  // out of the last scale, before the next item's
#pragma unroll                                                       // decode may write it
          for (int gi = 0; gi < kWideGroups; ++gi) {
            const float sl = last[gi * 16 + n];
#pragma unroll
            for (int i = 0; i < NTW; ++i) acc[gi][i] *= sl;
          }
        }
        lds_barrier();  // every wave is done with step k's buffer and has written step k + 1's
      }
    }
  }

  // lane (n, g) holds slots 4 g + j of each tile, row n of each group
#pragma unroll
  for (int i = 0; i < NTW; ++i) {
    const int t = t0 + wave + kWideWaves * i;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int slot = t * 16 + 4 * g + j;
      int ex = 0;
      if (p.a_max != nullptr) ex = row_exponent(p.a_max[p.a_row ? p.a_row[slot] : (uint32_t)slot]);
      if constexpr (kGlu) {
        OT* h = reinterpret_cast<OT*>(p.out) + (int64_t)slot * p.rows;
#pragma unroll
        for (int gi = 0; gi < kWideGroups / 2; ++gi) {
          const int row = rb * (8 * kWideGroups) + 16 * gi + n;
          const float v0 = __builtin_ldexpf(acc[gi][i][j], ex);
          const float v1 = __builtin_ldexpf(acc[gi + kWideGroups / 2][i][j], ex);
          if (row < p.rows) store_out<OT>(h + row, swiglu_f32(v0, v1));
        }
      } else {
        const uint32_t pr = p.slot_pair[slot];
        if (pr != 0xffffffffu) {
          OT* y = reinterpret_cast<OT*>(p.out) + (int64_t)pr * p.rows;
#pragma unroll
          for (int gi = 0; gi < kWideGroups; ++gi) {
            const int row = rb * (16 * kWideGroups) + 16 * gi + n;
            if (row < p.rows) store_out<OT>(y + row, __builtin_ldexpf(acc[gi][i][j], ex));
          }
        }
      }
    }
  }
}

template <int KIND, int MODE, typename OT>
__global__ __launch_bounds__(kWideThreads, kWideWavesSimd) void prompt_wide_kernel(PromptParams p) {
  static_assert(kWideGroups % kWideWaves == 0 && kWideGroups % 2 == 0, "whole groups of rows a wave");
  static_assert(MODE == PM_GLU || MODE == PM_SCATTER, "the SwiGLU and scatter forms");
  __shared__ __attribute__((aligned(16))) u32x4 wdec[2 * kWideBuf];
  __shared__ DirectTables<KIND> tab;
  __shared__ uint16_t chunks[kWideMaxTiles];
  __shared__ int scratch[kWideWaves];
  __shared__ float ratio[2 * kWideGroups * 16];
  __shared__ float last[kWideGroups * 16];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  {
    strata_mv::TableFetch<KIND> tf;
    strata_mv::fetch_tables<KIND, kWideThreads>(tf, tid);
    strata_mv::store_tables<KIND, kWideThreads>(tab, tf, tid);
  }
  const int total = wide_plan(p, chunks, scratch, tid);  // its barriers also publish the tables

  // items chunk by chunk, row block by row block, dealt to the workgroups in turn
  const int items = total * p.row_blocks;
  for (int it = blockIdx.x; it < items; it += gridDim.x) {
    const int c = it / p.row_blocks, rb = it % p.row_blocks;
    const int t0 = (int)chunks[c];
    const uint32_t e = p.tile_expert[t0];
    wide_item<KIND, MODE, OT, kWideTilesWave>(p, tab, wdec, ratio, last, e, t0, rb, wave, lane);  // a full chunk
  }
}

// Whether a launch splits into the wide form's full chunks and the chunked form's tails: the SwiGLU and scatter
// forms, a plan that fits, 16-byte rows of activations, and eight tiles an expert or more on average. A layer of
// 256 IQ3_S experts, Zipf top-8, bfloat16, whole (gate/up and down): 4096 tokens 442 against 430 TFLOPS, 8192
// tokens 513-518 against 486-489; at 2048 (4.4 tiles an expert) the same, 367-372 against 370-376: the heavy
// experts' full chunks of three were the chunked form's cheapest tiles, and what it keeps, the light experts'
// one-tile chunks, costs it as much as before.
template <int MODE>
inline bool wide_takes(const PromptParams& p) {
  return (MODE == PM_GLU || MODE == PM_SCATTER) && p.n_tiles <= kWideMaxTiles && ((uintptr_t)p.a & 15) == 0 &&
         p.n_tiles >= 8 * p.experts;
}

template <int KIND, int MODE, typename OT>
int launch_prompt_wide(PromptParams& p, hipStream_t s) {
  if constexpr (MODE == PM_GLU || MODE == PM_SCATTER) {
    constexpr int rows = wide_out_rows<MODE>();
    p.row_blocks = (p.rows + rows - 1) / rows;
    const int grid = kWidePerCU * strata_mv::device_cus() / kXcds * kXcds;
    if (grid < kXcds) return STRATA_ERR_SHAPE;
    hipLaunchKernelGGL((prompt_wide_kernel<KIND, MODE, OT>), dim3((unsigned)grid), dim3(kWideThreads), 0, s, p);
    STRATA_CHECK_LAUNCH();
    return STRATA_OK;
  } else {
    (void)p;
    (void)s;
    return STRATA_ERR_SHAPE;
  }
}

// A prompt launch: where the wide form takes it, the heavy experts' full chunks there, then the rest in the chunked
// form (skip_full); otherwise the chunked form alone.
template <int KIND, int MODE, typename OT>
int launch_prompt_split(PromptParams& p, hipStream_t s) {
  if constexpr (kStagedKind<KIND>) {  // the types the wide form decodes
    if (wide_takes<MODE>(p)) {
      const int rc = launch_prompt_wide<KIND, MODE, OT>(p, s);
      if (rc) return rc;
      p.skip_full = 1;
    }
  }
  return launch_prompt<KIND, MODE, OT>(p, s);
}

}  // namespace strata_prompt
