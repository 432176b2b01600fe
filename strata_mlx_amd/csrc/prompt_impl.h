// The prompt kernels: grouped dequant-matmuls over tiles of 16 slots, each tile one expert's, on CDNA4 MFMA, for
// IQ3_S, IQ3_XXS and Q2_0 rows of whole 256-weight steps and float16 activations (strata_mlx/blocks.py:583-694).
//
// c[s, :] = W[e(s)] . a[s, :]. A workgroup (4 waves) takes a chunk, up to NT = 3 consecutive tiles of one expert
// (a run of one expert's tiles is cut into chunks of NT from its first tile; the workgroup at a chunk's first tile
// works, the others exit at once), and a block of rows. Every wave holds two groups of 16 rows: in the SwiGLU form the same 16 rows of gate and of up, otherwise 32
// rows of one matrix. The expert's rows are decoded once for all tiles of the chunk, and the body is compiled for
// each chunk size, so no branch sits between the MFMAs.
//
// MFMA v_mfma_f32_16x16x32_f16: a (16 slots x 32) x w (32 x 16 rows), float32 sums. Lane (n, g) of a wave gives
// row n's weights, and it holds the fields of one run pair of the row (64 weights: runs 2g, 2g + 1 of each step of
// 256 columns), loaded straight from HBM into registers a step ahead. Run h's 32 weights are four MFMAs' worth (8 a
// lane each); the K order of an MFMA is therefore a permutation of the step's columns, and the slots' activations
// are read from LDS in that order. The weights reach the MFMA as exact float16 integers with the run's own scale
// folded in: IQ3_S's (1 + 2s) * grid (at most 465), IQ3_XXS's (2s + 1) * grid (at most 1922), Q2_0's d * (c - 1)
// (d times -1, 0, 1 or 2, exact unless |d| > 32752). What is common to a row's step (IQ3_S's d, IQ3_XXS's d / 4)
// multiplies the step's float32 sums, so nothing is rounded before the sums. Codebook entries come from LDS as
// float16 magnitudes; their signs are set in registers (no sign table in LDS).
//
// The activations of a step (16 slots x 256 columns of every tile of the chunk) go to LDS once for the workgroup.
// Slot s of the chunk reads activation row a_row[s] (the token, for gate and up) or row s (down, whose input is in
// slot order). Float16 activations only; bfloat16 ones are given as rows scaled into float16 by a power of two
// (strata_rows_to_f16: a row's largest magnitude into [2^14, 2^15)), with a_max holding each row's largest
// magnitude, and the sums are scaled back by that power exactly.
//
// Workgroup i runs on XCD i % 8. Windows of NT tiles go to the XCDs in turn, and every row block of a window's
// tiles runs on the window's XCD: the chunks (at most NT starting in a window) spread evenly over the XCDs, and a
// chunk's activations are read into one L2 (its workgroups are those of its first tile).
#pragma once
#include "direct_impl.h"

namespace strata_prompt {

using strata_mv::DirectTables;
using strata_mv::LaneOffsets;
using strata_mv::RunPair;

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 h2v __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kStep = 256;           // columns a K step: a 256-weight block of every row (four Q2_0 blocks)
constexpr int kPitch = kStep + 8;    // float16 a slot's step in LDS: 16 slots' 16-byte reads fall on distinct banks
constexpr int kXcds = 8;             // workgroup i runs on XCD i % 8
constexpr int kMinWaves = 3;         // waves a SIMD the kernels are built for (at most 168 VGPRs)

enum PromptMode : int { PM_C32 = 0, PM_GLU = 1, PM_SCATTER = 2 };

struct PromptParams {
  const uint8_t* blocks[2];     // the stacks: gate and up (SwiGLU form), else blocks[0]
  const f16* a;                 // float16 activations (a_rows x cols)
  const uint32_t* a_row;        // the activation row of each slot, or null (slot s reads row s)
  const uint32_t* a_max;        // scaled rows: each row's largest magnitude (float bits), or null
  const uint32_t* tile_expert;  // expert of each tile (>= experts: a tile to leave out)
  const uint32_t* slot_pair;    // scatter form: the output row of each slot (0xffffffff: none)
  void* out;                    // C32: float (slots x rows); SwiGLU: h (slots x rows); scatter: y (pairs x rows)
  int64_t experts, mat_bytes;
  int rows, cols, row_bytes, n_tiles, row_blocks;
  int skip_full;  // the full chunks of kFullChunk tiles are another launch's (prompt_wide.h): take the runs' tails
};

constexpr int kFullChunk = 16;  // tiles of a full chunk, taken by prompt_wide.h when PromptParams.skip_full is set

// The run's own scale, as a float16 pair: IQ3_S 1 + 2s, IQ3_XXS 2s + 1, Q2_0 d.
template <int KIND>
__device__ __forceinline__ h2v run_scale2(const RunPair<KIND>& f, int h, int g) {
  f16 m;
  if constexpr (KIND == K_IQ3_S) {
    m = (f16)(float)(1 + 2 * __builtin_amdgcn_ubfe((uint32_t)f.sc, 8 * (g & 1) + 4 * h, 4));
  } else if constexpr (KIND == K_IQ3_XXS) {
    m = (f16)(float)(1 + 2 * (f.aux[h] >> 28));
  } else {
    m = __builtin_bit_cast(f16, (uint16_t)f.d);
  }
  return h2v{m, m};
}

// The run's own scale folded into N packed float16 pairs of integers (exact, see above).
template <int KIND, int N>
__device__ __forceinline__ void fold_run(const RunPair<KIND>& f, int h, int g, uint32_t (&w)[N]) {
  const h2v m2 = run_scale2<KIND>(f, h, g);
#pragma unroll
  for (int i = 0; i < N; ++i) w[i] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2v, w[i]) * m2);
}

// What multiplies a row's whole step: IQ3_S d, IQ3_XXS d / 4 (strata_mlx/blocks.py:89-116); Q2_0 has none left.
template <int KIND>
__device__ __forceinline__ float step_scale(const RunPair<KIND>& f) {
  if constexpr (KIND == K_IQ3_S) return strata_mv::half_bits(f.d);
  if constexpr (KIND == K_IQ3_XXS) return strata_mv::half_bits(f.d) * 0.25f;
  return 1.0f;
}
template <int KIND>
constexpr bool has_step_scale() {
  return KIND == K_IQ3_S || KIND == K_IQ3_XXS;
}

// The signs of 8 weights (bits of s8, weight j at bit j) put on 8 float16 magnitudes (two codebook entries, whose sign
// bits are clear), in registers: s8 goes to both 16-bit halves of a word, a packed shift a word brings weight
// (2i, 2i + 1)'s bits to bit 15 of each half, and an and-or sets them.
__device__ __forceinline__ void put_signs(uint32_t s8, const u32x2& g0, const u32x2& g1, uint32_t* w) {
  typedef unsigned short us2 __attribute__((ext_vector_type(2)));
  const us2 d = __builtin_bit_cast(us2, s8 * 0x10001u);
  const uint32_t m0 = __builtin_bit_cast(uint32_t, (us2)(d << us2{15, 14}));
  const uint32_t m1 = __builtin_bit_cast(uint32_t, (us2)(d << us2{13, 12}));
  const uint32_t m2 = __builtin_bit_cast(uint32_t, (us2)(d << us2{11, 10}));
  const uint32_t m3 = __builtin_bit_cast(uint32_t, (us2)(d << us2{9, 8}));
  w[0] = (m0 & 0x80008000u) | g0[0];
  w[1] = (m1 & 0x80008000u) | g0[1];
  w[2] = (m2 & 0x80008000u) | g1[0];
  w[3] = (m3 & 0x80008000u) | g1[1];
}

// Group pair l (weights 8 l .. 8 l + 7) of run h of the lane's run pair g, IQ3_XXS, IQ3_S or Q2_0: 4 packed
// float16 pairs, the run's scale and signs folded in (exact). What the four group pairs of a run share is the same
// expression for each, computed once where they are unrolled together.
template <int KIND>
__device__ __forceinline__ void decode_folded4(const RunPair<KIND>& f, int h, int g, int l, uint32_t (&w)[4],
                                               const DirectTables<KIND>& t) {
  static_assert(KIND == K_IQ3_XXS || KIND == K_IQ3_S || KIND == K_Q2_0, "the staged types");
  if constexpr (KIND == K_Q2_0) {  // strata_mlx/blocks.py:58-68: code bytes 2 l, 2 l + 1 of the run, four (c - 1) each
    const uint32_t q = f.qs[2 * h + (l >> 1)];
    const u32x2 c0 = t.q2[(q >> (16 * (l & 1))) & 255];
    const u32x2 c1 = t.q2[(q >> (16 * (l & 1) + 8)) & 255];
    w[0] = c0[0];
    w[1] = c0[1];
    w[2] = c1[0];
    w[3] = c1[1];
  } else if constexpr (KIND == K_IQ3_XXS) {  // strata_mlx/blocks.py:103-116: groups 2l, 2l + 1, signs ksigns[7 bits of aux]
    const uint32_t q = f.qs[2 * h + (l >> 1)];
    const u32x2 g0 = t.grid[(q >> (16 * (l & 1))) & 255];
    const u32x2 g1 = t.grid[(q >> (16 * (l & 1) + 8)) & 255];
    const uint32_t s7 = __builtin_amdgcn_ubfe(f.aux[h], 7 * l, 7);
    // the parity in bit 7: the count's bit 0 (its bits 1-2 land in bits 8-9, which put_signs shifts out of both
    // 16-bit halves)
    const uint32_t s8 = s7 | ((uint32_t)__builtin_popcount(s7) << 7);
    put_signs(s8, g0, g1, w);
  } else {  // strata_mlx/blocks.py:89-102: groups 2l, 2l + 1, their ninth index bits from qh, signs byte l
    const uint32_t qs = f.qs[2 * h + (l >> 1)];
    const uint32_t qh = (f.qh >> (8 * h)) & 255;
    const uint32_t hb = (__builtin_amdgcn_ubfe(qh, 4 * (l >> 1), 4) * 0x204081u) & 0x01010101u;
    const uint32_t iw = __builtin_amdgcn_perm(hb, qs, (l & 1) ? 0x07030602u : 0x05010400u);
    const uint32_t three = 3;
    const u32x2 g0 = strata_mv::lds_entry(t.grid, strata_mv::word_shl<0>(iw, three));
    const u32x2 g1 = strata_mv::lds_entry(t.grid, strata_mv::word_shl<1>(iw, three));
    put_signs((f.sg[h] >> (8 * l)) & 255u, g0, g1, w);
  }
  fold_run<KIND, 4>(f, h, g, w);
}

// Run h of the lane's run pair g: 16 packed float16 pairs, the run's scale and signs folded in (exact).
template <int KIND>
__device__ __forceinline__ void decode_folded(const RunPair<KIND>& f, int h, int g, uint32_t (&w)[16],
                                              const DirectTables<KIND>& t) {
  if constexpr (KIND == K_IQ3_XXS || KIND == K_IQ3_S) {
#pragma unroll
    for (int l = 0; l < 4; ++l) {
      uint32_t w4[4];
      decode_folded4<KIND>(f, h, g, l, w4, t);
#pragma unroll
      for (int i = 0; i < 4; ++i) w[4 * l + i] = w4[i];
    }
  } else {
    strata_mv::decode_run<KIND>(f, h, g, w, t);
    fold_run<KIND, 16>(f, h, g, w);
  }
}

// Column (within the step) of the first of the 8 weights lane group g gives MFMA (h, q): run run_of(g, h), its
// weights 8q .. 8q + 7.
template <int KIND>
__device__ __forceinline__ int a_col(int g, int h, int q) {
  return 32 * strata_mv::run_of<KIND>(g, h) + 8 * q;
}

template <typename OT>
__device__ __forceinline__ void store_out(OT* p, float v) {
  *p = from_f32<OT>(v);
}

// silu(g) * u in float32, as mlx-lm's swiglu computes it on the float32 products (strata_mlx/blocks.py:692).
__device__ __forceinline__ float swiglu_f32(float g, float u) {
  const float s = 1.0f / (1.0f + expf(-g));
  return (g * s) * u;
}

// lane (n, g) holds slots 4g + j of each tile, for rows row0 and row1
template <int MODE, typename OT, int NTC>
__device__ __forceinline__ void write_chunk(const PromptParams& p, const f32x4 (&acc)[2][NTC], int t0, int g,
                                            int row0, int row1) {
#pragma unroll
  for (int i = 0; i < NTC; ++i) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int slot = (t0 + i) * 16 + 4 * g + j;
      float v0 = acc[0][i][j], v1 = acc[1][i][j];
      if (p.a_max != nullptr) {
        const uint32_t r = p.a_row ? p.a_row[slot] : (uint32_t)slot;
        const int ex = row_exponent(p.a_max[r]);
        v0 = __builtin_ldexpf(v0, ex);
        v1 = __builtin_ldexpf(v1, ex);
      }
      if constexpr (MODE == PM_C32) {
        float* c = reinterpret_cast<float*>(p.out) + (int64_t)slot * p.rows;
        if (row0 < p.rows) c[row0] = v0;
        if (row1 < p.rows) c[row1] = v1;
      } else if constexpr (MODE == PM_GLU) {
        if (row0 < p.rows)
          store_out<OT>(reinterpret_cast<OT*>(p.out) + (int64_t)slot * p.rows + row0, swiglu_f32(v0, v1));
      } else {
        const uint32_t pr = p.slot_pair[slot];
        if (pr != 0xffffffffu) {
          OT* y = reinterpret_cast<OT*>(p.out) + (int64_t)pr * p.rows;
          if (row0 < p.rows) store_out<OT>(y + row0, v0);
          if (row1 < p.rows) store_out<OT>(y + row1, v1);
        }
      }
    }
  }
}

// One chunk of exactly NTC tiles (NTC at compile time: no per-tile branches between the MFMAs).
template <int KIND, int MODE, typename OT, int WAVES, int NTC>
__device__ __forceinline__ void run_chunk(const PromptParams& p, const DirectTables<KIND>& tab,
                                          f16* a_lds, uint32_t e, int t0, int rb, int tid,
                                          int wave) {
  constexpr int kThreadsWg = 64 * WAVES;
  constexpr bool kGlu = MODE == PM_GLU;
  constexpr int kRowsWave = kGlu ? 16 : 32;
  constexpr int kChunks = NTC * 16 * (kStep / 8);  // 16-byte pieces of the chunk's activations a step
  constexpr int kLoads = kChunks / kThreadsWg;      // a thread's
  static_assert(kChunks % kThreadsWg == 0, "whole pieces a thread");
  const int lane = tid & 63;

  // the lane's rows and fields
  const int n = lane & 15, g = lane >> 4;
  const int r0 = rb * kRowsWave * WAVES + wave * kRowsWave;
  const int row0 = r0 + n, row1 = kGlu ? r0 + n : r0 + 16 + n;
  const uint8_t* mat0 = p.blocks[0] + (int64_t)e * p.mat_bytes;
  const uint8_t* mat1 = kGlu ? p.blocks[1] + (int64_t)e * p.mat_bytes : mat0;
  const uint32_t off0 = (uint32_t)min(row0, p.rows - 1) * (uint32_t)p.row_bytes;
  const uint32_t off1 = (uint32_t)min(row1, p.rows - 1) * (uint32_t)p.row_bytes;
  const LaneOffsets<KIND> o = strata_mv::lane_offsets<KIND>(g);
  const int nsteps = p.cols / kStep;
  const uint32_t step_bytes = (uint32_t)(p.row_bytes / nsteps);

  // the thread's pieces of the activations: (tile, slot, piece) -> global row and LDS place
  const f16* arow[kLoads];
  int adst[kLoads];
#pragma unroll
  for (int q = 0; q < kLoads; ++q) {
    const int c = tid + q * kThreadsWg;
    const int i = c / (16 * (kStep / 8)), m = (c / (kStep / 8)) % 16, piece = c % (kStep / 8);
    const int slot = (t0 + i) * 16 + m;
    const uint32_t r = p.a_row ? p.a_row[slot] : (uint32_t)slot;
    arow[q] = p.a + (int64_t)r * p.cols + 8 * piece;
    adst[q] = (i * 16 + m) * kPitch + 8 * piece;
  }
  u32x4 av[kLoads];
#pragma unroll
  for (int q = 0; q < kLoads; ++q) av[q] = *reinterpret_cast<const u32x4*>(arow[q]);

  RunPair<KIND> f[2][2];  // [step parity][row group]
  strata_mv::load_fields<KIND>(mat0, off0, o, f[0][0]);
  strata_mv::load_fields<KIND>(mat1, off1, o, f[0][1]);

  f32x4 acc[2][NTC];
#pragma unroll
  for (int i = 0; i < NTC; ++i) acc[0][i] = acc[1][i] = f32x4{0.f, 0.f, 0.f, 0.f};

  for (int kb = 0; kb < nsteps; kb += 2) {
#pragma unroll
    for (int sp = 0; sp < 2; ++sp) {
      const int k = kb + sp;
      if (k < nsteps) {
        // the next step's fields (past the last step, the last again: unconditional loads)
        const uint32_t nx = (uint32_t)min(k + 1, nsteps - 1) * step_bytes;
        strata_mv::load_fields<KIND>(mat0, off0 + nx, o, f[sp ^ 1][0]);
        strata_mv::load_fields<KIND>(mat1, off1 + nx, o, f[sp ^ 1][1]);
        __syncthreads();  // every wave has read the last step's activations (and the tables are written)
#pragma unroll
        for (int q = 0; q < kLoads; ++q) *reinterpret_cast<u32x4*>(a_lds + adst[q]) = av[q];
        if (k + 1 < nsteps) {
#pragma unroll
          for (int q = 0; q < kLoads; ++q) av[q] = *reinterpret_cast<const u32x4*>(arow[q] + (k + 1) * kStep);
        }
        __syncthreads();

        f32x4 part[2][NTC];
#pragma unroll
        for (int i = 0; i < NTC; ++i) part[0][i] = part[1][i] = f32x4{0.f, 0.f, 0.f, 0.f};
        auto read_a = [&](f16x8 (&a8)[4][NTC], int h, int q) {
#pragma unroll
          for (int i = 0; i < NTC; ++i)
            a8[q][i] = *reinterpret_cast<const f16x8*>(a_lds + (i * 16 + n) * kPitch + a_col<KIND>(g, h, q));
        };
        auto mfma_group = [&](const f16x8 (&a8)[NTC], const uint32_t* w0, const uint32_t* w1) {
          const f16x8 b0 = __builtin_bit_cast(f16x8, u32x4{w0[0], w0[1], w0[2], w0[3]});
          const f16x8 b1 = __builtin_bit_cast(f16x8, u32x4{w1[0], w1[1], w1[2], w1[3]});
#pragma unroll
          for (int i = 0; i < NTC; ++i) {
            f32x4& p0 = has_step_scale<KIND>() ? part[0][i] : acc[0][i];
            f32x4& p1 = has_step_scale<KIND>() ? part[1][i] : acc[1][i];
            p0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a8[i], b0, p0, 0, 0, 0);
            p1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a8[i], b1, p1, 0, 0, 0);
          }
        };
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          f16x8 a8[4][NTC];
          if constexpr (NTC >= 3 && (KIND == K_IQ3_S || KIND == K_IQ3_XXS)) {  // a group pair at a time, as staged
            read_a(a8, h, 0);
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              uint32_t w0[4], w1[4];
              decode_folded4<KIND>(f[sp][0], h, g, q, w0, tab);
              decode_folded4<KIND>(f[sp][1], h, g, q, w1, tab);
              if (q + 1 < 4) read_a(a8, h, q + 1);
              mfma_group(a8[q], w0, w1);
            }
          } else {  // the first two groups' activations read ahead of the decode, so their latency passes under it
#pragma unroll
            for (int q = 0; q < 2; ++q) read_a(a8, h, q);
            uint32_t w0[16], w1[16];
            decode_folded<KIND>(f[sp][0], h, g, w0, tab);
            decode_folded<KIND>(f[sp][1], h, g, w1, tab);
#pragma unroll
            for (int q = 2; q < 4; ++q) read_a(a8, h, q);
#pragma unroll
            for (int q = 0; q < 4; ++q) mfma_group(a8[q], w0 + 4 * q, w1 + 4 * q);
          }
        }
        if constexpr (has_step_scale<KIND>()) {
          const float s0 = step_scale<KIND>(f[sp][0]), s1 = step_scale<KIND>(f[sp][1]);
#pragma unroll
          for (int i = 0; i < NTC; ++i) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              acc[0][i][j] = __builtin_fmaf(s0, part[0][i][j], acc[0][i][j]);
              acc[1][i][j] = __builtin_fmaf(s1, part[1][i][j], acc[1][i][j]);
            }
          }
        }
      }
    }
  }

  write_chunk<MODE, OT, NTC>(p, acc, t0, g, row0, row1);
}


// The staged form of run_chunk (IQ3_S, IQ3_XXS, Q2_0): the rows' bytes of a step go to LDS by gfx950's direct loads
// (global_load_lds_dword: lane l's dword lands at M0 + 4 l), each wave instruction a contiguous 256-byte piece of
// two or three rows, and each lane reads its fields from there. Loaded straight into registers (run_chunk), each of
// a lane's field loads touches the cache lines of 16 rows at once, and the texture-address unit and the L1 tag
// lookups, not HBM, set the pace (Q2_0's kernels with their field loads in registers: TA busy 70 %, TD 84 % of the
// launch; staged, the 512-token Q2_0 chunk went from 186 to 222-228 TFLOPS).
//
// A wave stages its own rows: two groups of 16 (SwiGLU form: its gate rows, then its up rows), each row a slot of
// 112 bytes holding the dwords from the one with the step's first byte to the one with its last (a step of 110 or
// 98 bytes starts two bytes into a dword at odd steps; rows are whole dwords; Q2_0's step, four 18-byte blocks, is
// 72 bytes from a dword, in a slot of 80). Those dwords lie within the stack
// whenever its base and a row's bytes are multiples of 4 (the launch checks). LDS reads are naturally aligned
// (16-byte reads at multiples of 16, 8-byte at multiples of 8: misaligned ones run about 14 times slower), and a
// field that starts 2 or 4 bytes past such a boundary is put together in registers (v_alignbyte).
//
// One row buffer a wave: the next step's rows are asked for as soon as this step's fields are in registers, and
// arrive while they are decoded. Chunks of up to three tiles take one activation buffer and two workgroup barriers a
// step (the kernels built for chunks of at most two take two buffers and one barrier; two buffers of three tiles
// would leave two workgroups a CU). The loads are inline assembly, so the compiler places no wait of its own for
// them: the one wait (vmcnt(0)) comes at the top of each step, and the barriers wait only for LDS (a __syncthreads
// would also wait for the next step's rows). The LDS (42-44 KB) and the registers (159-167) leave three workgroups
// on a CU; at two (a third row buffer, or the IQ3_XXS codebook with its signs folded in, 32 KB) or at four (128
// registers, spilled) the kernel ran slower.
template <int KIND>
constexpr bool kStagedKind = KIND == K_IQ3_S || KIND == K_IQ3_XXS || KIND == K_Q2_0;
template <int KIND>
constexpr int kStepBytes = KIND == K_IQ3_S ? 110 : KIND == K_IQ3_XXS ? 98 : 72;  // Q2_0: four 18-byte blocks
template <int KIND>
constexpr int kSlotDwords = (kStepBytes<KIND> + 2) / 4;  // dwords a row's step spans: 28, 25, 18
template <int KIND>
constexpr int kSlotPitch = KIND == K_Q2_0 ? 20 : 28;     // dwords a row's slot (112 bytes; Q2_0 80)
template <int KIND>
constexpr int kGroupLoads = 16 * kSlotPitch<KIND> / 64;  // wave instructions a group of 16 rows: 7 (Q2_0 5)
template <int KIND>
constexpr int kGroupBytes = 256 * kGroupLoads<KIND>;     // a group's buffer

// lane l's dword at base + voff into LDS at lds + 4 l (the wave's LDS address in M0, which the load reads when
// it issues). M0 is the compiler's register: its value is kept in an SGPR and put back after the load, so the
// assembly changes no register the compiler does not know of. (The compiler's own global_load_lds builtin adds
// waits for every load in flight before LDS reads it cannot tell apart: prompt 171-173 against 179-180 TFLOPS.)
__device__ __forceinline__ void dma_dword(const uint8_t* base, uint32_t voff, uint32_t lds) {
  uint32_t saved;
  asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dword %2, %3\n\ts_mov_b32 m0, %0"
               : "=&s"(saved)
               : "s"(lds), "v"(voff), "s"(base)
               : "memory");
}
__device__ __forceinline__ void wait_loads() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

typedef uint32_t u32x4a16 __attribute__((ext_vector_type(4), aligned(16)));
typedef uint32_t u32x2a8 __attribute__((ext_vector_type(2), aligned(8)));
template <typename T>
__device__ __forceinline__ T lds_at(const uint8_t* base, uint32_t off) {  // off a multiple of sizeof(T)
  const __attribute__((address_space(3))) uint8_t* b = (const __attribute__((address_space(3))) uint8_t*)base;
  return *(const __attribute__((address_space(3))) T*)(b + off);
}
// 16 bytes at a0 + SH (a0 a multiple of 16; SH 2 or 4)
template <int SH>
__device__ __forceinline__ u32x4 lds_16(const uint8_t* base, uint32_t a0) {
  const u32x4a16 w = lds_at<u32x4a16>(base, a0);
  const uint32_t w4 = lds_at<uint32_t>(base, a0 + 16);
  if constexpr (SH == 4) return u32x4{w[1], w[2], w[3], w4};
  return u32x4{__builtin_amdgcn_alignbyte(w[1], w[0], SH), __builtin_amdgcn_alignbyte(w[2], w[1], SH),
               __builtin_amdgcn_alignbyte(w[3], w[2], SH), __builtin_amdgcn_alignbyte(w4, w[3], SH)};
}
// 8 bytes at a0 + SH (a0 a multiple of 8; SH 2 or 4)
template <int SH>
__device__ __forceinline__ u32x2 lds_8(const uint8_t* base, uint32_t a0) {
  const u32x2a8 w = lds_at<u32x2a8>(base, a0);
  const uint32_t w2 = lds_at<uint32_t>(base, a0 + 8);
  if constexpr (SH == 4) return u32x2{w[1], w2};
  return u32x2{__builtin_amdgcn_alignbyte(w[1], w[0], SH), __builtin_amdgcn_alignbyte(w2, w[1], SH)};
}
// lane g's fields from a staged row slot whose step starts S bytes in (S = 0 or 2): the fields at the offsets of
// lane_offsets (d @0, qs @2 + 16 g; IQ3_S qh @66 + 2 g, signs @74 + 8 g, scale @106 + 2 (g / 2); IQ3_XXS aux
// @66 + 8 g)
template <int KIND, int S>
__device__ __forceinline__ void lds_fields(const uint8_t* slot, int g, RunPair<KIND>& f) {
  const uint32_t gg = (uint32_t)g;
  if constexpr (KIND == K_Q2_0) {  // a step is 72 bytes from a dword (S unused): block g's d @18 g, qs @18 g + 2
    const uint32_t o = 18u * gg, q = o + 2u, a = q & ~3u, sh = q & 3u;
    f.d = lds_at<uint16_t>(slot, o);
    uint32_t dw[5];
#pragma unroll
    for (int k = 0; k < 5; ++k) dw[k] = lds_at<uint32_t>(slot, a + 4u * k);
    f.qs = u32x4{__builtin_amdgcn_alignbyte(dw[1], dw[0], sh), __builtin_amdgcn_alignbyte(dw[2], dw[1], sh),
                 __builtin_amdgcn_alignbyte(dw[3], dw[2], sh), __builtin_amdgcn_alignbyte(dw[4], dw[3], sh)};
  } else {
    f.d = lds_at<uint16_t>(slot, S);
    f.qs = lds_16<S + 2>(slot, 16 * gg);
    if constexpr (KIND == K_IQ3_S) {
      f.qh = lds_at<uint16_t>(slot, S + 66 + 2 * gg);
      f.sg = lds_8<S + 2>(slot, 72 + 8 * gg);
      f.sc = lds_at<uint16_t>(slot, S + 106 + 2 * (gg >> 1));
    } else {
      f.aux = lds_8<S + 2>(slot, 64 + 8 * gg);
    }
  }
}

// Activation buffers of the staged form: two (one barrier a step) up to chunks of two tiles; for longer chunks one,
// which keeps the LDS at three workgroups a CU (a second barrier a step waits for its writes).
template <int NT>
constexpr int activation_buffers() {
  return NT <= 2 ? 2 : 1;
}

template <int KIND, int MODE, typename OT, int WAVES, int NT, int NTC>
__device__ __forceinline__ void run_chunk_staged(const PromptParams& p, const DirectTables<KIND>& tab,
                                                 f16* a_lds, uint8_t* w_lds, uint32_t e, int t0, int rb, int tid,
                                                 int wave) {
  constexpr int kThreadsWg = 64 * WAVES;
  constexpr bool kGlu = MODE == PM_GLU;
  constexpr int kRowsWave = kGlu ? 16 : 32;
  constexpr int kChunks = NTC * 16 * (kStep / 8);
  constexpr int kLoads = kChunks / kThreadsWg;
  static_assert(kChunks % kThreadsWg == 0, "whole pieces a thread");
  static_assert(kStagedKind<KIND>, "staged rows: IQ3_S, IQ3_XXS, Q2_0");
  constexpr int kSB = kStepBytes<KIND>, kDW = kSlotDwords<KIND>, kGL = kGroupLoads<KIND>, kPitchDw = kSlotPitch<KIND>;
  constexpr int kGB = kGroupBytes<KIND>;
  constexpr int kABuf = NT * 16 * kPitch;  // float16: an activation buffer
  constexpr int kABufs = activation_buffers<NT>();
  const int lane = tid & 63;

  const int n = lane & 15, g = lane >> 4;
  const int r0 = rb * kRowsWave * WAVES + wave * kRowsWave;
  const int row0 = r0 + n, row1 = kGlu ? r0 + n : r0 + 16 + n;
  const uint8_t* mat[2] = {p.blocks[0] + (int64_t)e * p.mat_bytes,
                           (kGlu ? p.blocks[1] : p.blocks[0]) + (int64_t)e * p.mat_bytes};
  const int grow[2] = {r0, kGlu ? r0 : r0 + 16};  // first row of each group
  const int nsteps = p.cols / kStep;

  // the lane's dword of each staging load: row q of the group, dword d of its slot (the slot's spare dwords: the
  // row's last dword again)
  uint32_t voff[2][kGL];
#pragma unroll
  for (int grp = 0; grp < 2; ++grp)
#pragma unroll
    for (int i = 0; i < kGL; ++i) {
      const int f = 64 * i + lane;
      const int q = f / kPitchDw, d = min(f % kPitchDw, kDW - 1);
      voff[grp][i] = (uint32_t)min(grow[grp] + q, p.rows - 1) * (uint32_t)p.row_bytes + 4u * (uint32_t)d;
    }
  const uint32_t w_base = (uint32_t)(uintptr_t)w_lds;
  auto stage = [&](int k) {
    const uint32_t first = (uint32_t)(k * kSB) & ~3u;  // the dword holding the step's first byte
#pragma unroll
    for (int grp = 0; grp < 2; ++grp) {
      const uint8_t* base = mat[grp] + first;
      const uint32_t dst = __builtin_amdgcn_readfirstlane(w_base + (uint32_t)((wave * 2 + grp) * kGB));
#pragma unroll
      for (int i = 0; i < kGL; ++i) dma_dword(base, voff[grp][i], dst + 256u * i);
    }
  };

  const f16* arow[kLoads];
  int adst[kLoads];
#pragma unroll
  for (int q = 0; q < kLoads; ++q) {
    const int c = tid + q * kThreadsWg;
    const int i = c / (16 * (kStep / 8)), m = (c / (kStep / 8)) % 16, piece = c % (kStep / 8);
    const int slot = (t0 + i) * 16 + m;
    const uint32_t r = p.a_row ? p.a_row[slot] : (uint32_t)slot;
    arow[q] = p.a + (int64_t)r * p.cols + 8 * piece;
    adst[q] = (i * 16 + m) * kPitch + 8 * piece;
  }
  u32x4 av[kLoads];
#pragma unroll
  for (int q = 0; q < kLoads; ++q) av[q] = *reinterpret_cast<const u32x4*>(arow[q]);
  if constexpr (kABufs == 2) {
#pragma unroll
    for (int q = 0; q < kLoads; ++q) *reinterpret_cast<u32x4*>(a_lds + adst[q]) = av[q];
  }
  stage(0);
  if (kABufs == 2 && nsteps > 1) {
#pragma unroll
    for (int q = 0; q < kLoads; ++q) av[q] = *reinterpret_cast<const u32x4*>(arow[q] + kStep);
  }

  f32x4 acc[2][NTC];
#pragma unroll
  for (int i = 0; i < NTC; ++i) acc[0][i] = acc[1][i] = f32x4{0.f, 0.f, 0.f, 0.f};

  for (int kb = 0; kb < nsteps; kb += 2) {
#pragma unroll
    for (int sp = 0; sp < 2; ++sp) {
      const int k = kb + sp;
      if (k < nsteps) {
        // two buffers: this wave's rows of step k and its activation pieces of step k + 1 are in, every wave's
        // activations of step k are written and every wave is done with step k - 1; one buffer: the pieces of
        // step k are in, and every wave is done reading step k - 1's
        wait_loads();
        lds_barrier();
        if constexpr (kABufs == 2) {
          if (k + 1 < nsteps) {
#pragma unroll
            for (int q = 0; q < kLoads; ++q) *reinterpret_cast<u32x4*>(a_lds + (sp ^ 1) * kABuf + adst[q]) = av[q];
          }
        } else {
#pragma unroll
          for (int q = 0; q < kLoads; ++q) *reinterpret_cast<u32x4*>(a_lds + adst[q]) = av[q];
        }
        RunPair<KIND> f[2];
#pragma unroll
        for (int grp = 0; grp < 2; ++grp) {
          const uint8_t* slot = reinterpret_cast<const uint8_t*>(w_lds) + (wave * 2 + grp) * kGB +
                                4 * kPitchDw * n;
          if (sp == 0)  // k even: the step starts at a dword; odd: 2 bytes in (kSB is 2 mod 4)
            lds_fields<KIND, 0>(slot, g, f[grp]);
          else
            lds_fields<KIND, 2>(slot, g, f[grp]);
        }
        if (k + 1 < nsteps) {  // the rows of step k + 1 into the same buffer, once this step's fields are read
          asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
          stage(k + 1);
        }
        if (k + kABufs < nsteps) {
#pragma unroll
          for (int q = 0; q < kLoads; ++q) av[q] = *reinterpret_cast<const u32x4*>(arow[q] + (k + kABufs) * kStep);
        }
        if constexpr (kABufs == 1) lds_barrier();  // every wave's activations of step k are written
        const f16* ab = a_lds + (kABufs == 2 ? sp * kABuf : 0);

        f32x4 part[2][NTC];
#pragma unroll
        for (int i = 0; i < NTC; ++i) part[0][i] = part[1][i] = f32x4{0.f, 0.f, 0.f, 0.f};
        // Two forms of a run's work. Whole: both row groups' runs decoded at once, two MFMA groups' activations
        // read ahead of the decode and two after it. Interleaved (chunks of three tiles, whose registers the whole
        // form overruns): group pair q of both runs decoded just before MFMA group q, whose activations are read
        // while group q - 1 multiplies.
        constexpr bool kInterleaved = NTC >= 3;
        auto read_a = [&](f16x8 (&a8)[4][NTC], int h, int q) {
#pragma unroll
          for (int i = 0; i < NTC; ++i)
            a8[q][i] = *reinterpret_cast<const f16x8*>(ab + (i * 16 + n) * kPitch + a_col<KIND>(g, h, q));
        };
        auto mfma_group = [&](const f16x8 (&a8)[NTC], const uint32_t* w0, const uint32_t* w1) {
          const f16x8 b0 = __builtin_bit_cast(f16x8, u32x4{w0[0], w0[1], w0[2], w0[3]});
          const f16x8 b1 = __builtin_bit_cast(f16x8, u32x4{w1[0], w1[1], w1[2], w1[3]});
#pragma unroll
          for (int i = 0; i < NTC; ++i) {
            part[0][i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a8[i], b0, part[0][i], 0, 0, 0);
            part[1][i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a8[i], b1, part[1][i], 0, 0, 0);
          }
        };
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          f16x8 a8[4][NTC];
          if constexpr (kInterleaved) {
            read_a(a8, h, 0);
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              uint32_t w0[4], w1[4];
              decode_folded4<KIND>(f[0], h, g, q, w0, tab);
              decode_folded4<KIND>(f[1], h, g, q, w1, tab);
              if (q + 1 < 4) read_a(a8, h, q + 1);
              mfma_group(a8[q], w0, w1);
            }
          } else {
#pragma unroll
            for (int q = 0; q < 2; ++q) read_a(a8, h, q);
            uint32_t w0[16], w1[16];
            decode_folded<KIND>(f[0], h, g, w0, tab);
            decode_folded<KIND>(f[1], h, g, w1, tab);
#pragma unroll
            for (int q = 2; q < 4; ++q) read_a(a8, h, q);
#pragma unroll
            for (int q = 0; q < 4; ++q) mfma_group(a8[q], w0 + 4 * q, w1 + 4 * q);
          }
        }
        const float s0 = step_scale<KIND>(f[0]), s1 = step_scale<KIND>(f[1]);
#pragma unroll
        for (int i = 0; i < NTC; ++i) {
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            acc[0][i][j] = __builtin_fmaf(s0, part[0][i][j], acc[0][i][j]);
            acc[1][i][j] = __builtin_fmaf(s1, part[1][i][j], acc[1][i][j]);
          }
        }
      }
    }
  }
  write_chunk<MODE, OT, NTC>(p, acc, t0, g, row0, row1);
}

template <int KIND, int MODE, typename OT, int WAVES, int NT, bool STAGED>
__global__ __launch_bounds__(64 * WAVES, kMinWaves) void prompt_kernel(PromptParams p) {
  constexpr int kThreadsWg = 64 * WAVES;
  constexpr bool kStagedHere = STAGED && kStagedKind<KIND>;
  __shared__ __attribute__((aligned(16))) uint8_t w_lds[kStagedHere ? WAVES * 2 * kGroupBytes<KIND> : 16];
  __shared__ DirectTables<KIND> tab;
  __shared__ __attribute__((aligned(16))) f16 a_lds[(kStagedHere ? activation_buffers<NT>() : 1) * NT * 16 * kPitch];

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);

  // (tile, row block) of this workgroup: windows of NT tiles dealt to the XCDs in turn (every row block of a
  // window's tiles on one XCD), so that the chunks, which start at the windows, spread evenly
  const int L = blockIdx.x, xcd = L % kXcds, s = L / kXcds;
  const int per_window = NT * p.row_blocks;
  const int w = kXcds * (s / per_window) + xcd, j = (s / p.row_blocks) % NT, rb = s % p.row_blocks;
  const int t0 = w * NT + j;
  if (t0 >= p.n_tiles) return;
  const uint32_t e = p.tile_expert[t0];
  if (e >= (uint64_t)p.experts) return;  // a tile nothing fills: left out
  // A run of one expert's consecutive tiles is cut into chunks of NT from its first tile: this workgroup works if
  // the run's tiles before t0 are a multiple of NT. The first round looks at the 64 tiles before t0 (lane l at
  // t0 - 1 - l), which settles every run of up to 64 tiles; each later one at the next 256 (lane l at
  // t0 - 1 - before - 64 j - l, j = 0..3, four loads in flight at once), so that a run of thousands of tiles takes
  // a few rounds. (Four loads from the first round on cost 1 % at the usual routings.)
  int before;
  {
    const int t = t0 - 1 - (tid & 63);
    const uint64_t m = __ballot(t < 0 || p.tile_expert[t] != e);
    before = m != 0 ? __builtin_ctzll(m) : 64;
  }
  for (bool more = before == 64; more;) {
    bool other[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int t = t0 - 1 - before - 64 * j - (tid & 63);
      other[j] = t < 0 || p.tile_expert[t] != e;
    }
    int seen = 256;  // tiles of the run among those looked at, before the first other one
#pragma unroll
    for (int j = 3; j >= 0; --j) {
      const uint64_t m = __ballot(other[j]);
      if (m != 0) seen = 64 * j + __builtin_ctzll(m);
    }
    before += seen;
    more = seen == 256;
  }
  if (p.skip_full) {  // a run's first floor(L / 16) * 16 tiles are full chunks, another launch's; the tail is this one's
    // t0's block of 16 from the run's first tile is full if every tile from t0 to its end names e (lanes 0-15)
    const int left = kFullChunk - before % kFullChunk, t = t0 + (tid & 63);
    const bool ok = (tid & 63) >= left || (t < p.n_tiles && p.tile_expert[t] == e);
    if (__ballot(!ok) == 0) return;  // a full chunk's tile
    before %= kFullChunk;            // the tail's tiles before t0
  }
  if (__builtin_amdgcn_readfirstlane(before) % NT != 0) return;  // a tile of a chunk that starts before it
  int nt = 1;
#pragma unroll
  for (int i = 1; i < NT; ++i)
    if (t0 + i < p.n_tiles && nt == i && p.tile_expert[t0 + i] == e) nt = i + 1;
  nt = __builtin_amdgcn_readfirstlane(nt);

  {  // the codebooks, read after the K loop's first barrier
    strata_mv::TableFetch<KIND> tf;
    strata_mv::fetch_tables<KIND, kThreadsWg>(tf, tid);
    strata_mv::store_tables<KIND, kThreadsWg>(tab, tf, tid);
  }
  static_assert(NT >= 2 && NT <= 8, "chunks of up to two to eight tiles");
  // the body compiled for each chunk size up to NT: no branch between the MFMAs
  auto go = [&](auto ntc) {
    constexpr int NTC = decltype(ntc)::value;
    if constexpr (NTC <= NT) {
      if constexpr (kStagedHere)
        run_chunk_staged<KIND, MODE, OT, WAVES, NT, NTC>(p, tab, a_lds, w_lds, e, t0, rb, tid, wave);
      else
        run_chunk<KIND, MODE, OT, WAVES, NTC>(p, tab, a_lds, e, t0, rb, tid, wave);
    }
  };
  switch (nt) {
    case 1: go(std::integral_constant<int, 1>()); break;
    case 2: go(std::integral_constant<int, 2>()); break;
    case 3: go(std::integral_constant<int, 3>()); break;
    case 4: go(std::integral_constant<int, 4>()); break;
    case 5: go(std::integral_constant<int, 5>()); break;
    case 6: go(std::integral_constant<int, 6>()); break;
    case 7: go(std::integral_constant<int, 7>()); break;
    default: go(std::integral_constant<int, 8>()); break;
  }
}

template <int MODE>
constexpr int rows_per_wg(int waves) {
  return (MODE == PM_GLU ? 16 : 32) * waves;
}

// Whether the prompt kernels take a stack: a type they decode, rows of whole 256-weight steps.
inline bool prompt_takes(int kind, int64_t cols) {
  return (kind == K_IQ3_S || kind == K_IQ3_XXS || kind == K_Q2_0) && cols % kStep == 0 && cols > 0;
}

constexpr int kWaves = 4;
constexpr int kTiles = 3;  // tiles a chunk at most (an expert's rows decoded once for them)
constexpr bool kStaged = true;  // rows through LDS by direct loads (run_chunk_staged)

template <int KIND, int MODE, typename OT>
int launch_prompt(PromptParams& p, hipStream_t s) {
  constexpr int rpw = rows_per_wg<MODE>(kWaves);
  p.row_blocks = (p.rows + rpw - 1) / rpw;
  const int64_t tiles = (p.n_tiles + kXcds * kTiles - 1) / (kXcds * kTiles) * (kXcds * kTiles);
  const int64_t grid = tiles * p.row_blocks;
  if (grid <= 0) return STRATA_OK;
  if (grid > 0x7fffffff) return STRATA_ERR_SHAPE;
  // staged rows read whole dwords: the stacks' bases and a row's bytes multiples of 4
  const bool staged = kStaged && kStagedKind<KIND> && ((uintptr_t)p.blocks[0] & 3) == 0 && ((uintptr_t)p.blocks[1] & 3) == 0 &&
                      p.row_bytes % 4 == 0 && p.mat_bytes % 4 == 0;
  if (staged)
    hipLaunchKernelGGL((prompt_kernel<KIND, MODE, OT, kWaves, kTiles, true>), dim3((unsigned)grid), dim3(64 * kWaves),
                       0, s, p);
  else
    hipLaunchKernelGGL((prompt_kernel<KIND, MODE, OT, kWaves, kTiles, false>), dim3((unsigned)grid), dim3(64 * kWaves),
                       0, s, p);
  STRATA_CHECK_LAUNCH();
  return STRATA_OK;
}

}  // namespace strata_prompt
