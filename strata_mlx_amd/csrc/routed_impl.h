// Routed gate and up with the SwiGLU, and the routed one-matrix product (down), in IQ3_S and Q2_0 for decode:
// the matvecs of a mixture-of-experts layer at a few tokens (strata_mlx/blocks.py:958-975 with the SwiGLU of its
// down call, :222-236), each as one persistent launch.
//
// What a launch of direct_decode_kernel spends at this shape is mostly fixed cost: a chain of dependent loads
// before the first row byte is asked for (the parameters, the pair's expert, the mode's branches), a prologue and
// an epilogue for every four row steps, and 1.5 rounds of single-shot waves. Here one workgroup of sixteen waves
// sits on each CU for the whole launch, and a wave takes UPW units (a unit: row r of the gate matrix and row r of
// the up matrix of one pair), all known when it starts: their experts are read at once, the rows of up to three
// units are in flight together (a fourth goes out once the first is decoded), and the units' sums are written at
// the end by one lane each (one SwiGLU evaluation a wave, not one a unit).
//
// Order of the loads. The codebook and the token are asked for first and the workgroup barrier waits for them
// alone; the rows go out after it. A CU's loads return in the order they were asked for, so rows asked for
// before the barrier put every wave's codebook load behind the other waves' rows: the barrier then passed at
// 3.4-9 us into the launch instead of about 1 us (per-wave timestamps), and nothing was decoded until then. With a
// barrier that waits for nothing once every wave has asked for its table entry and token (so that all of those
// come before any row), the rows before the table still made the one-token gate/up launch slower, 17.0 against
// 14.0 us.
// For the same reason nothing of the decode may be moved above the barrier (opaque(): the compiler would
// otherwise compute the codebook addresses there and wait for the rows at the barrier).
//
// The codebook sits in LDS with its signs folded in: entry s << 9 | g is grid entry g (nine index bits) with
// sign bit b of s flipping weight b, four float16 integers, 8192 entries of 8 bytes. A group of four weights is
// then one LDS read, its address one shift of a 16-bit word whose low byte is the index byte and whose high byte
// is the ninth index bit and the four sign bits, put together by v_perm from the fields as loaded. (With a
// separate 16-entry sign table, a group was two reads, two address shifts and two XORs.) The table and the token
// take 72 KB of LDS; at more than 64 VGPRs a CU holds one such workgroup.
//
// Lane j of a wave holds run pair j of a row (64 weights, the same 128 bytes of the token for every unit); the
// gate row's partial sums and the up row's meet in one exchange of halves and then within the halves.
//
// Several tokens (pairs / share of them, up to 8): every pair is its own unit, and the tokens sit in LDS beside
// the codebook; a wave's units are consecutive rows of a pair, and it reads its token's 128 bytes a lane from LDS
// once a pair. Q2_0 takes the same kernels with a 256-entry table of a code byte's four weights (c - 1) in place
// of the codebook, and d for a lane's block.
#pragma once

#include "topk.h"
// Included by direct_impl.h ahead of the dispatch (it uses that file's fields, offsets and reductions).

namespace strata_mv {

constexpr int kGluThreads = 1024;  // sixteen waves a workgroup, one workgroup a CU
constexpr int kGluWaves = kGluThreads / 64;
// Q6_K and Q8_0 (a run pair's fields take 18 registers) at eight waves a workgroup: the registers for three units'
// rows a wave (at sixteen waves, two units' rows spilled). Q4_K with a float32 token (mode 3, ONE32) too: a
// 4096 x 4096 matrix is 2048 units of two rows, which at one a wave fill every CU only at eight waves a workgroup.
template <int KIND, int MODE = 0>
constexpr int glu_threads() {
  return KIND == K_Q6_K || KIND == K_Q8_0 || (KIND == K_Q4_K && MODE == 3) ? 512 : kGluThreads;
}
constexpr int kGluGroupsPerCU = 1;
constexpr int kGluMaxUnits = 16;   // units a wave (straight-line code); more units: more waves
constexpr int kGluMaxTokens = 8;   // tokens in LDS

// What a type brings to these kernels: its LDS table (built by the workgroup), the fields of a lane's run pair
// (64 weights), their loads, the lane's share of a row's sum, and how many units' fields fit in registers at
// once. This form is the linear types' (Q4_K, Q6_K, Q8_0): the direct kernel's register decode, no table.
template <int KIND>
struct Routed {
  static constexpr int kEntries = 1;
  static constexpr int kBuffers = glu_threads<KIND>() < kGluThreads ? 3 : 2;
  typedef RunPair<KIND> Fields;
  static __device__ __forceinline__ uint64_t fetch(int) { return 0; }
  static __device__ __forceinline__ void fill(u32x2*, int, uint64_t) {}
  static __device__ __forceinline__ void load(const uint8_t* row, int j, Fields& f) {
    load_fields<KIND>(row, 0u, lane_offsets<KIND>(j), f);
  }
  // xs: the lane's sums of x for biased runs (x_sums of both runs, kXSums a run), the same for every unit
  static constexpr int kPrepSums = 2 * kXSums<KIND>;  // xs: the sums of x of both runs (x_sums)
  static __device__ __forceinline__ void prep_x(uint32_t* x, float* xs) {
    if constexpr (kBiasedRuns<KIND>) {
      x_sums<KIND>(x, xs);
      x_sums<KIND>(x + 16, xs + kXSums<KIND>);
    }
  }
  static __device__ __forceinline__ float pair_sum_lds(const Fields& f, int j, const uint32_t* x, const float* xs,
                                                       const u32x2* tab) {
    return pair_sum(f, j, x, xs, tab);
  }
  static __device__ __forceinline__ float pair_sum(const Fields& f, int j, const uint32_t* x, const float* xs,
                                                   const u32x2* tab) {
    const DirectTables<KIND>& t = *reinterpret_cast<const DirectTables<KIND>*>(tab);  // unused by these types
    float s = 0.0f;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      uint32_t w[16];
      const RunScale rs = decode_run<KIND>(f, h, j, w, t);
      s += apply_run<KIND>(rs, w, x + 16 * h, xs + kXSums<KIND> * h);
    }
    return s;
  }
  // the same against x_a + x_b (a float32 token as two float16 parts): each run decoded once
  static __device__ __forceinline__ float pair_sum2(const Fields& f, int j, const uint32_t* xa, const uint32_t* xb,
                                                    const float* xsa, const float* xsb, const u32x2* tab) {
    const DirectTables<KIND>& t = *reinterpret_cast<const DirectTables<KIND>*>(tab);
    float s = 0.0f;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      uint32_t w[16];
      const RunScale rs = decode_run<KIND>(f, h, j, w, t);
      s += apply_run<KIND>(rs, w, xa + 16 * h, xsa + kXSums<KIND> * h) +
           apply_run<KIND>(rs, w, xb + 16 * h, xsb + kXSums<KIND> * h);
    }
    return s;
  }
};

template <>
struct Routed<K_IQ3_S> {
  static constexpr int kEntries = 8192;  // 512 grid entries x 16 sign nibbles
  static constexpr int kBuffers = 3;
  typedef RunPair<K_IQ3_S> Fields;
  // the codebook entry thread tid expands (asked for before anything else)
  static __device__ __forceinline__ uint64_t fetch(int tid) { return kIq3sHalfGrid.v[tid & 511]; }
  // entry s << 9 | g: grid entry g under sign nibble s (bit b flips weight b); thread tid writes half the nibbles
  // of entry tid % 512
  static __device__ __forceinline__ void fill(u32x2* tab, int tid, uint64_t entry) {
    const uint32_t lo32 = (uint32_t)entry, hi32 = (uint32_t)(entry >> 32);
    const int half = (tid >> 9) & 1;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int s = 8 * half + i;
      const uint32_t m0 = ((i & 1) ? 0x8000u : 0u) | ((i & 2) ? 0x80000000u : 0u);
      const uint32_t m1 = ((i & 4) ? 0x8000u : 0u) | (half ? 0x80000000u : 0u);
      tab[s * 512 + (tid & 511)] = u32x2{lo32 ^ m0, hi32 ^ m1};
    }
  }
  // run pair j of the row at `row` (d @0, qs[64] @2, qh[8] @66, signs[32] @74, scales[4] @106 of each 110-byte
  // block); the loads take the row as a scalar base and a 32-bit lane offset
  static __device__ __forceinline__ void load(const uint8_t* row, int j, Fields& f) {
    const uint32_t b = (uint32_t)(j >> 2) * 110, jj = (uint32_t)j & 3;
    f.d = load_at<uint16_t>(row, b);
    f.qs = load_at<u32x4>(row + 2, b + 16 * jj);
    f.qh = load_at<uint16_t>(row + 66, b + 2 * jj);
    f.sg = load_at<u32x2>(row + 74, b + 8 * jj);
    f.sc = load_at<uint16_t>(row + 106, b + 2 * (jj >> 1));
  }
  // Run h (0, 1): its 32 weights from the signed codebook, times 32 activations (16 packed pairs). Group l's
  // word: the index byte qs[l] low, the ninth bit and the sign nibble of group l high. The ninth bits of the even
  // groups (bits 0, 2, 4, 6 of the run's qh byte) go to bit 0 of bytes 0..3 by one multiply (the products' other
  // bits never reach bits 0, 8, 16, 24), the sign nibbles of the even groups are the low nibbles of the run's
  // four sign bytes; the odd groups take bits 1, 3, 5, 7 and the high nibbles.
  static __device__ __forceinline__ float run(const Fields& f, int h, const uint32_t* x, const u32x2* tab) {
    const uint32_t q0 = f.qs[2 * h], q1 = f.qs[2 * h + 1];
    const uint32_t hb = (uint32_t)f.qh >> (8 * h);
    const uint32_t sg = f.sg[h];
    const uint32_t he = (((hb & 0x55u) * 0x41041u) & 0x01010101u) | ((sg & 0x0F0F0F0Fu) << 1);
    const uint32_t ho = ((((hb >> 1) & 0x55u) * 0x41041u) & 0x01010101u) | ((sg >> 3) & 0x1E1E1E1Eu);
    const uint32_t w02 = __builtin_amdgcn_perm(he, q0, 0x05020400u), w13 = __builtin_amdgcn_perm(ho, q0, 0x05030401u);
    const uint32_t w46 = __builtin_amdgcn_perm(he, q1, 0x07020600u), w57 = __builtin_amdgcn_perm(ho, q1, 0x07030601u);
    const uint32_t three = 3;
    const uint32_t a[8] = {word_shl<0>(w02, three), word_shl<0>(w13, three), word_shl<1>(w02, three),
                           word_shl<1>(w13, three), word_shl<0>(w46, three), word_shl<0>(w57, three),
                           word_shl<1>(w46, three), word_shl<1>(w57, three)};
    uint32_t w[16];
#pragma unroll
    for (int l = 0; l < 8; ++l) {
      const u32x2 v = lds_entry(tab, a[l]);
      w[2 * l] = v[0];
      w[2 * l + 1] = v[1];
    }
    return dot16x2(w, x + 16 * h);
  }
  // lane j's share of a row: its two runs, each times its scale d (1 + 2 s)
  static constexpr int kPrepSums = 0;
  static __device__ __forceinline__ void prep_x(uint32_t*, float*) {}
  static __device__ __forceinline__ float pair_sum_lds(const Fields& f, int j, const uint32_t* x, const float* xs,
                                                       const u32x2* tab) {
    return pair_sum(f, j, x, xs, tab);
  }
  static __device__ __forceinline__ float pair_sum(const Fields& f, int j, const uint32_t* x, const float*,
                                                   const u32x2* tab) {
    const float d = half_bits(f.d);
    const uint32_t sc = (uint32_t)f.sc >> (8 * (j & 1));
    const float s0 = d * (float)(1 + 2 * (sc & 15u)), s1 = d * (float)(1 + 2 * ((sc >> 4) & 15u));
    return s0 * run(f, 0, x, tab) + s1 * run(f, 1, x, tab);
  }
};

template <>
struct Routed<K_Q2_0> {
  static constexpr int kEntries = 256;  // a code byte's four weights c - 1 as float16
  static constexpr int kBuffers = 3;
  typedef RunPair<K_Q2_0> Fields;
  static __device__ __forceinline__ uint64_t fetch(int) { return 0; }
  static __device__ __forceinline__ void fill(u32x2* tab, int tid, uint64_t) {
    if (tid < 256) {
      const uint32_t b = (uint32_t)tid;
      tab[tid] = u32x2{pack_h2((float)(b & 3) - 1.0f, (float)((b >> 2) & 3) - 1.0f),
                       pack_h2((float)((b >> 4) & 3) - 1.0f, (float)(b >> 6) - 1.0f)};
    }
  }
  // run pair j = block j of the row (d @0, qs[16] @2 of each 18-byte block; weight k in bits 2 (k % 4) of byte
  // k / 4, strata_mlx/blocks.py:58-68)
  static __device__ __forceinline__ void load(const uint8_t* row, int j, Fields& f) {
    const uint32_t b = (uint32_t)j * 18;
    f.d = load_at<uint16_t>(row, b);
    f.qs = load_at<u32x4>(row + 2, b);
  }
  static __device__ __forceinline__ float run(const Fields& f, int h, const uint32_t* x, const u32x2* tab) {
    const uint32_t q0 = f.qs[2 * h], q1 = f.qs[2 * h + 1];
    const uint32_t three = 3;
    const uint32_t a[8] = {byte_shl<0>(q0, three), byte_shl<1>(q0, three), byte_shl<2>(q0, three),
                           byte_shl<3>(q0, three), byte_shl<0>(q1, three), byte_shl<1>(q1, three),
                           byte_shl<2>(q1, three), byte_shl<3>(q1, three)};
    uint32_t w[16];
#pragma unroll
    for (int l = 0; l < 8; ++l) {
      const u32x2 v = lds_entry(tab, a[l]);
      w[2 * l] = v[0];
      w[2 * l + 1] = v[1];
    }
    return dot16x2(w, x + 16 * h);
  }
  // down (routed_down_kernel): the table
  static __device__ __forceinline__ float pair_sum_lds(const Fields& f, int, const uint32_t* x, const float*,
                                                       const u32x2* tab) {
    return half_bits(f.d) * (run(f, 0, x, tab) + run(f, 1, x, tab));
  }
  // Gate and up (routed_glu_kernel) decode in registers, no table: byte b of a run (codes c0..c3 of weights
  // 4b .. 4b + 3) goes to bytes 0 and 2 of a word (one v_perm), and two and-ors with 0x6400 give the float16
  // integers 1024 + c0, 1024 + 4 c1 and 1024 + 16 c2, 1024 + 64 c3 (exact). The token was divided weight by
  // weight by 1, 4, 16, 64 (prep_x: exact powers of two), so each product is 1024 x' + c x, and the run's
  // 1024 sum x' + sum x (in xs) takes off the 1024 and the 1 of c - 1. A lookup table's 8-byte reads at random
  // entries left half the LDS cycles to bank conflicts.
  static constexpr int kPrepSums = 2;  // xs: one float a run
  static __device__ __forceinline__ void prep_x(uint32_t* x, float* xs) {
    typedef _Float16 h2v __attribute__((ext_vector_type(2)));
    const uint32_t ones[16] = {0x3C003C00u, 0x3C003C00u, 0x3C003C00u, 0x3C003C00u, 0x3C003C00u, 0x3C003C00u,
                               0x3C003C00u, 0x3C003C00u, 0x3C003C00u, 0x3C003C00u, 0x3C003C00u, 0x3C003C00u,
                               0x3C003C00u, 0x3C003C00u, 0x3C003C00u, 0x3C003C00u};
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const float sx = dot_n<16>(ones, x + 16 * h);
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const h2v m = (i & 1) ? h2v{(_Float16)0.0625f, (_Float16)0.015625f} : h2v{(_Float16)1.0f, (_Float16)0.25f};
        x[16 * h + i] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2v, x[16 * h + i]) * m);
      }
      xs[h] = 1024.0f * dot_n<16>(ones, x + 16 * h) + sx;
    }
  }
  static __device__ __forceinline__ float pair_sum(const Fields& f, int, const uint32_t* x, const float* xs,
                                                   const u32x2*) {
    // the masks and 0x6400 0x6400 in registers: an and-or takes three, and a VALU instruction of three operands
    // here takes no literal and one scalar register at most
    uint32_t m01, m23, base;
    asm("v_mov_b32 %0, 0x000C0003" : "=v"(m01));
    asm("v_mov_b32 %0, 0x00C00030" : "=v"(m23));
    asm("v_mov_b32 %0, 0x64006400" : "=v"(base));
    float s = 0.0f;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      uint32_t w[16];
#pragma unroll
      for (int l = 0; l < 8; ++l) {
        const uint32_t q = f.qs[2 * h + (l >> 2)], k = (uint32_t)(l & 3);
        const uint32_t dup = __builtin_amdgcn_perm(q, q, 0x0C000C00u | (k << 16) | k);  // byte k at bytes 0, 2
        w[2 * l] = (dup & m01) | base;
        w[2 * l + 1] = (dup & m23) | base;
      }
      s += dot16x2(w, x + 16 * h) - xs[h];
    }
    return half_bits(f.d) * s;
  }
};

// GLU1: gate and up of one token (a unit: row r of each); GLUN: the same at several tokens, in LDS; ONE: one
// matrix and one token, no routing (a unit: rows 2 i and 2 i + 1); ONE32: ONE with a float32 token and float32
// products (the token scaled by a power of two into float16 and split into two float16 parts, x = hi + lo).
enum GluMode : int { GLU1 = 0, GLUN = 1, ONE = 2, ONE32 = 3 };

struct GluParams {
  const uint8_t* gate;  // ONE: the matrix
  const uint8_t* up;
  const uint32_t* idx;  // expert of each pair (ONE: none)
  const u32x4* x;       // the tokens: 4096 float16 each, as 512 pieces of 16 bytes (ONE32: 4096 float32, 1024)
  f16* out_gate;        // gate . x (may be null); ONE: the product
  f16* out_up;          // up . x (may be null)
  f16* h;               // silu(gate . x) * (up . x)
  int64_t mat_bytes;
  uint32_t experts;
  int rows, row_bytes, pairs, share, tokens, waves;
  // units: u = a * nb + b, (a, b) = (pair, row) for one token, (row, pair) for several; from a wave's unit to its
  // next, (a, b) moves by (wave_a, wave_b) with a carry
  int na, nb, wave_a, wave_b;
  // the shared expert in the same launch (one token, routed_glu_kernel's SHARED form): its gate and up (Q4_K,
  // s_rows x 4096) and silu(gate . x) * (up . x) out; its unit r (row r of each) is wave r * waves / s_rows's
  const uint8_t* s_gate;
  const uint8_t* s_up;
  f16* s_h;
  f16* s_g;  // the shared expert's gate . x, or null
  f16* s_u;  // its up . x, or null
  int s_rows, s_row_bytes;
  // the choice of experts in the launch (routed_glu_kernel's ROUTE form, one token): the router's logits (float32,
  // r_rows of them: the experts' r_experts first, then rows such as a shared expert's gate), the pairs' experts and
  // weights out (idx is the launch's own choice: top `pairs` of the experts' logits, their softmax) and the rows
  // past the experts' rounded to float16 (or null)
  const float* r_logits;
  uint32_t* r_idx;
  float* r_w;
  f16* r_extra;
  int r_rows, r_experts;
};

// A token's piece c (16 bytes: columns 8 c .. 8 c + 7) in LDS: slot c with its low three bits XORed with the
// next three, so that the eight lanes of one LDS cycle of a 16-byte read (pieces 8 j + i of lanes j) fall on
// distinct banks.
__device__ __forceinline__ int glu_x_slot(int j, int i) { return 8 * j + (i ^ (j & 7)); }
__device__ __forceinline__ int x_piece_slot(int c) { return glu_x_slot(c >> 3, c & 7); }

// The unit's two rows decoded and multiplied (gate and up, or rows 2 i and 2 i + 1), and their sums met over the
// wave: the first row's total and the second's, the same in every lane (read into scalars).
template <int KIND, bool TWO = false>
__device__ __forceinline__ void glu_unit(typename Routed<KIND>::Fields (&f)[2], int lane, const uint32_t* x,
                                         const uint32_t* x2, const float* xs, const float* xs2, const u32x2* tab,
                                         float& gate, float& up) {
  opaque(f[0]);  // nothing of the decode is done before the workgroup barrier (it would wait for these rows there)
  opaque(f[1]);
  float g, u;
  if constexpr (TWO) {
    g = Routed<KIND>::pair_sum2(f[0], lane, x, x2, xs, xs2, tab);
    u = Routed<KIND>::pair_sum2(f[1], lane, x, x2, xs, xs2, tab);
  } else {
    g = Routed<KIND>::pair_sum(f[0], lane, x, xs, tab);
    u = Routed<KIND>::pair_sum(f[1], lane, x, xs, tab);
  }
  // lanes 0-31 the first row's partial sums two at a time, lanes 32-63 the second's; then within the halves
  float v = sum_swapped(g, u, 32);
  v = sum_swapped(v, v, 16);
  v += lanes_apart(v, 8);
  v += lanes_apart(v, 4);
  v += lanes_apart(v, 2);
  v += lanes_apart(v, 1);
  gate = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__float_as_int(v), 0));
  up = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__float_as_int(v), 32));
}

// ROUTE (one token, 256 experts at most): the pairs' experts are chosen in the launch from the router's logits, by
// wave 0 of every workgroup while the table and the token go to LDS (the same choice as top_k's); workgroup 0 writes
// it out for the down and combine launches. It spares the router's launch the count and the choice at its end.
template <int KIND, int UPW, int MODE, bool SHARED = false, bool ROUTE = false>
__global__ __launch_bounds__((glu_threads<KIND, MODE>()), (glu_threads<KIND, MODE>() / 256)) void routed_glu_kernel(
    GluParams p) {
  constexpr int kGluThreads = glu_threads<KIND, MODE>(), kGluWaves = kGluThreads / 64;
  typedef Routed<KIND> R;
  typedef typename R::Fields Fields;
  constexpr bool kOne = MODE == ONE || MODE == ONE32;
  // units whose rows are in registers at once: ONE32 holds two parts of the token, SHARED the shared expert's unit
  constexpr int kMaxBuffers = MODE == ONE32 ? 1 : SHARED ? R::kBuffers - 1 : R::kBuffers;
  constexpr int kBuffers = UPW < kMaxBuffers ? UPW : kMaxBuffers;  // units whose rows are in registers at once
  constexpr int kTokens = MODE == GLUN ? kGluMaxTokens : MODE == ONE32 ? 2 : 1;
  // one block of LDS, the table first: its entries then sit below 64 KB, where a lookup's address is the entry's
  // offset alone (placed after eight tokens' 64 KB, every lookup took an add); the tokens at a multiple of 16
  // bytes (a 16-byte LDS read at any other address runs many times slower)
  constexpr int kTabBytes = (8 * R::kEntries + 15) / 16 * 16;
  __shared__ __attribute__((aligned(16))) uint8_t lds[kTabBytes + 16 * 512 * kTokens + 4 * kGluWaves];
  u32x2* const tab = reinterpret_cast<u32x2*>(lds);
  u32x4* const xs = reinterpret_cast<u32x4*>(lds + kTabBytes);
  uint32_t* const wmax = reinterpret_cast<uint32_t*>(lds + kTabBytes + 16 * 512 * kTokens);
  const int tid = threadIdx.x, lane = tid & 63;
  const int gw = blockIdx.x * kGluWaves + __builtin_amdgcn_readfirstlane(tid >> 6);

  // what the workgroup shares, asked for first: the table entry this thread expands and pieces of the tokens
  // (ONE32: quarters of float32 pieces, four values each: 1024 of them over the workgroup)
  const uint64_t entry = R::fetch(tid);
  static_assert(!ROUTE || MODE == GLU1, "the choice in the launch: one token");
  __shared__ uint32_t route_idx[ROUTE ? 64 : 1];
  __shared__ float route_w[ROUTE ? 64 : 1];
  float route_v[4];  // ROUTE: wave 0's logits, lane l holding experts l, l + 64, l + 128, l + 192
  if constexpr (ROUTE) {
    if (tid < 64) {
#pragma unroll
      for (int i = 0; i < 4; ++i) route_v[i] = p.r_logits[min(i * 64 + lane, p.r_experts - 1)];
    }
  }
  constexpr int kPieceLoads = MODE == ONE32 ? 1024 / kGluThreads : (512 * kTokens + kGluThreads - 1) / kGluThreads;
  u32x4 xpiece[kPieceLoads];
#pragma unroll
  for (int k = 0; k < kPieceLoads; ++k)
    xpiece[k] = p.x[MODE == ONE32 ? tid + k * kGluThreads : min(tid + k * kGluThreads, 512 * p.tokens - 1)];

  // the wave's units (pair, row) and whether each is live; ONE: row is the unit's first row (2 i), pair 0
  int pair[UPW], row[UPW];
  bool live[UPW];
  {
    // GLUN: a wave's units consecutive, pair by pair (its token read once a pair); else gw, gw + waves, ...
    const int u0 = MODE == GLUN ? gw * UPW : gw;
    int a = u0 / p.nb, b = u0 - a * p.nb;
#pragma unroll
    for (int k = 0; k < UPW; ++k) {
      live[k] = a < p.na;
      const int pr = a, r = b;
      if constexpr (kOne) {
        pair[k] = 0;
        row[k] = live[k] ? 2 * b : 0;  // past the last unit: the first rows again, nothing written
      } else {
        pair[k] = live[k] ? pr : p.pairs - 1;  // past the last unit: the last pair's last row again, nothing written
        row[k] = live[k] ? r : p.rows - 1;
      }
      b += MODE == GLUN ? 1 : p.wave_b;
      a += MODE == GLUN ? 0 : p.wave_a;
      if (b >= p.nb) {
        b -= p.nb;
        ++a;
      }
    }
  }
  uint32_t expert[UPW];
  bool bad[UPW];
#pragma unroll
  for (int k = 0; k < UPW; ++k) {
    if constexpr (kOne || ROUTE) {  // ROUTE: the experts are known after the workgroup barrier below
      bad[k] = false;
      expert[k] = 0u;
    } else {
      const uint32_t e = p.idx[pair[k]];
      bad[k] = e >= p.experts;
      expert[k] = bad[k] ? 0u : e;  // a pair naming no expert reads expert 0's rows and writes NaN
    }
  }
  auto issue = [&](int k, Fields(&f)[2]) {
    if constexpr (kOne) {
      const uint8_t* r0 = p.gate + (int64_t)row[k] * p.row_bytes;
      R::load(r0, lane, f[0]);
      R::load(row[k] + 1 < p.rows ? r0 + p.row_bytes : r0, lane, f[1]);  // an odd last row: the same row twice
    } else {
      const int64_t off = (int64_t)expert[k] * p.mat_bytes + (int64_t)row[k] * p.row_bytes;
      R::load(p.gate + off, lane, f[0]);
      R::load(p.up + off, lane, f[1]);
    }
    asm volatile("" ::: "memory");  // the units' loads go out in unit order
  };

  // ONE32 with a type that has no table (Q4_K, Q6_K, Q8_0): the rows go out as soon as every wave has asked for
  // its token pieces (a barrier that waits for nothing puts all of those ahead of the first row), and arrive while
  // the token's largest magnitude is found over the workgroup and the token is scaled into LDS (Q4_K 4096 x 4096:
  // 6.63 -> 5.73 us). With a table, rows ahead of it held its fill back (see the top of this file); in the other
  // modes, whose token only goes to LDS, the same order was slower (Q6_K 12288 x 4096: 13.0 -> 14.4 us).
  constexpr bool kEarlyRows = MODE == ONE32 && R::kEntries == 1;
  Fields f[kBuffers][2];
  if constexpr (kEarlyRows) {
    asm volatile("s_barrier" ::: "memory");
#pragma unroll
    for (int k = 0; k < kBuffers; ++k) issue(k, f[k]);
  }
  R::fill(tab, tid, entry);
  int ex = 0;  // ONE32: the token was divided by 2^ex
  if constexpr (MODE == ONE32) {
    // the token's largest magnitude over the workgroup, then the power of two that puts it in [2^14, 2^15)
    uint32_t m = 0;
#pragma unroll
    for (int k = 0; k < kPieceLoads; ++k)
#pragma unroll
      for (int i = 0; i < 4; ++i) m = max(m, xpiece[k][i] & 0x7fffffffu);
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) m = max(m, (uint32_t)__shfl_xor((int)m, d));
    if (lane == 0) wmax[tid >> 6] = m;
    if constexpr (kEarlyRows)
      asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");  // the LDS written; the rows stay in flight
    else
      __syncthreads();
#pragma unroll
    for (int w = 0; w < kGluWaves; ++w) m = max(m, wmax[w]);
    ex = row_exponent(m);
    // quarter c's four values as hi = float16(v / 2^ex) and lo = float16(v / 2^ex - hi): half of float16 piece c / 2
#pragma unroll
    for (int k = 0; k < kPieceLoads; ++k) {
      const int c = tid + k * kGluThreads;
      uint32_t hi[2], lo[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const float a = __builtin_ldexpf(__uint_as_float(xpiece[k][2 * i]), -ex);
        const float b = __builtin_ldexpf(__uint_as_float(xpiece[k][2 * i + 1]), -ex);
        const f16 ha = from_f32<f16>(a), hb = from_f32<f16>(b);
        const f16 la = from_f32<f16>(a - (float)ha), lb = from_f32<f16>(b - (float)hb);
        hi[i] = (uint32_t)__builtin_bit_cast(uint16_t, ha) | ((uint32_t)__builtin_bit_cast(uint16_t, hb) << 16);
        lo[i] = (uint32_t)__builtin_bit_cast(uint16_t, la) | ((uint32_t)__builtin_bit_cast(uint16_t, lb) << 16);
      }
      u32x2* h2 = reinterpret_cast<u32x2*>(xs + x_piece_slot(c >> 1)) + (c & 1);
      u32x2* l2 = reinterpret_cast<u32x2*>(xs + 512 + x_piece_slot(c >> 1)) + (c & 1);
      *h2 = u32x2{hi[0], hi[1]};
      *l2 = u32x2{lo[0], lo[1]};
    }
  } else {
#pragma unroll
    for (int k = 0; k < kPieceLoads; ++k) {
      const int c = min(tid + k * kGluThreads, 512 * p.tokens - 1);  // threads past the pieces write one again
      xs[(c >> 9) * 512 + x_piece_slot(c & 511)] = xpiece[k];
    }
  }
  if constexpr (ROUTE) {  // wave 0: the top `pairs` experts and their softmax, into LDS; workgroup 0's out as well
    if (tid < 64) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (i * 64 + lane >= p.r_experts) route_v[i] = -INFINITY;
      strata_topk::top_k_row<4>(route_v, p.r_experts, p.pairs, lane, route_idx, route_w);
      if (blockIdx.x == 0) {
        if (lane < p.pairs) {
          p.r_idx[lane] = route_idx[lane];
          p.r_w[lane] = route_w[lane];
        }
        for (int e = lane; p.r_extra != nullptr && e < p.r_rows - p.r_experts; e += 64)
          p.r_extra[e] = from_f32<f16>(p.r_logits[p.r_experts + e]);
      }
    }
  }
  if constexpr (kEarlyRows)
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  else
    __syncthreads();
  if constexpr (ROUTE) {  // a row of NaN logits chooses no expert (index 0xffffffff): read as a pair naming none
#pragma unroll
    for (int k = 0; k < UPW; ++k) {
      const uint32_t e = route_idx[pair[k]];
      bad[k] = e >= p.experts;
      expert[k] = bad[k] ? 0u : e;
    }
  }
  // lane j's activations: the 32 columns of each of its two runs
  uint32_t x[32], x2[MODE == ONE32 ? 32 : 1];
  auto read_x = [&](int t, uint32_t* dst) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int r = run_of<KIND>(lane, h);
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const u32x4 c = xs[t * 512 + x_piece_slot(4 * r + v)];
#pragma unroll
        for (int i = 0; i < 4; ++i) dst[16 * h + 4 * v + i] = c[i];
      }
    }
  };
  if constexpr (MODE != GLUN) read_x(0, x);
  if constexpr (MODE == ONE32) read_x(1, x2);
  if constexpr (!kEarlyRows) {
#pragma unroll
    for (int k = 0; k < kBuffers; ++k) issue(k, f[k]);
  }
  // the shared expert's unit of this wave (SHARED), if it has one: the first s with s * waves >= gw * s_rows,
  // if s * waves < (gw + 1) * s_rows; its rows asked for with the routed units' first ones, decoded after them
  typedef Routed<K_Q4_K> RS;
  typename RS::Fields fs[2];
  int s_unit = -1;
  if constexpr (SHARED) {
    static_assert(MODE == GLU1, "the shared expert at one token");
    const int64_t num = (int64_t)gw * p.s_rows;
    const int64_t su = (num + p.waves - 1) / p.waves;
    if (su < p.s_rows && su * p.waves < num + p.s_rows) s_unit = (int)su;
    if (s_unit >= 0) {
      const int64_t off = (int64_t)s_unit * p.s_row_bytes;
      RS::load(p.s_gate + off, lane, fs[0]);
      RS::load(p.s_up + off, lane, fs[1]);
    }
  }
  // what the type takes from the token once for every unit (the linear types' sums of x, Q2_0's scaled token and
  // its sums), after the rows are asked for (taken before, they held the loads back until the token's LDS reads
  // were in); GLUN: at each new pair, below
  float xsum[R::kPrepSums + 1], xsum2[R::kPrepSums + 1];
  if constexpr (MODE != GLUN) R::prep_x(x, xsum);
  if constexpr (MODE == ONE32) R::prep_x(x2, xsum2);

  // lane k collects unit k's two totals
  float gv = 0.0f, uv = 0.0f;
#pragma unroll
  for (int k = 0; k < UPW; ++k) {
    if constexpr (MODE == GLUN) {
      if (k == 0 || pair[k] != pair[k - 1]) {
        read_x(pair[k] / p.share, x);
        R::prep_x(x, xsum);
      }
    }
    float g, u;
    glu_unit<KIND, MODE == ONE32>(f[k % kBuffers], lane, x, x2, xsum, xsum2, tab, g, u);
    if (k + kBuffers < UPW) issue(k + kBuffers, f[k % kBuffers]);
    gv = lane == k ? g : gv;
    uv = lane == k ? u : uv;
  }

  // lane k writes unit k: gate, up and silu(gate) * up as mlx-lm rounds it; ONE: the two rows' products
  bool w_live = false, w_bad = false;
  int w_pair = 0, w_row = 0;
#pragma unroll
  for (int k = 0; k < UPW; ++k) {
    if (lane == k) {
      w_live = live[k];
      w_bad = bad[k];
      w_pair = pair[k];
      w_row = row[k];
    }
  }
  if (lane < UPW && w_live) {
    if constexpr (MODE == ONE32) {
      float* out = reinterpret_cast<float*>(p.out_gate);
      out[w_row] = __builtin_ldexpf(gv, ex);
      if (w_row + 1 < p.rows) out[w_row + 1] = __builtin_ldexpf(uv, ex);
    } else if constexpr (MODE == ONE) {
      p.out_gate[w_row] = from_f32<f16>(gv);
      if (w_row + 1 < p.rows) p.out_gate[w_row + 1] = from_f32<f16>(uv);
    } else {
      const int64_t o = (int64_t)w_pair * p.rows + w_row;
      f16 gq = from_f32<f16>(gv), uq = from_f32<f16>(uv), hq;
      if (w_bad) {
        gq = uq = hq = (f16)__builtin_nanf("");
      } else {
        hq = from_f32<f16>(swiglu_rounded<f16>(gq, uq));
      }
      if (p.out_gate != nullptr) p.out_gate[o] = gq;
      if (p.out_up != nullptr) p.out_up[o] = uq;
      p.h[o] = hq;
    }
  }
  if constexpr (SHARED) {
    if (s_unit >= 0) {
      // Q4_K's lane j takes runs 2 j and 2 j + 1, as these types do; Q2_0 scaled its registers: read them again
      static_assert(KIND == K_IQ3_S || KIND == K_Q2_0, "the routed type's runs are Q4_K's");
      if constexpr (KIND == K_Q2_0) read_x(0, x);
      float sx[RS::kPrepSums + 1];
      RS::prep_x(x, sx);
      float g, u;
      glu_unit<K_Q4_K>(fs, lane, x, x, sx, sx, tab, g, u);
      if (lane == 0) {
        const f16 gq = from_f32<f16>(g), uq = from_f32<f16>(u);
        p.s_h[s_unit] = from_f32<f16>(swiglu_rounded<f16>(gq, uq));
        if (p.s_g != nullptr) p.s_g[s_unit] = gq;
        if (p.s_u != nullptr) p.s_u[s_unit] = uq;
      }
    }
  }
}

// Down (and any one-matrix routed product) on rows of 1536 or 2560 inputs: 8 lanes take a row, lane m its run
// pairs m, m + 8, ... (S of them), so a wave holds 8 rows (a unit). A workgroup (one a CU) takes consecutive units
// of one pair, whose token sits in LDS beside the table; the rows go out after the barrier, as in
// routed_glu_kernel, and a row's sum meets over its 8 lanes by three DPP steps.
struct DownParams {
  const uint8_t* blocks;
  const uint32_t* idx;
  const f16* x;  // pairs / share tokens of 512 S float16
  f16* out;
  int64_t mat_bytes;
  uint32_t experts;
  int rows, row_bytes, pairs, share;
  int groups_per_pair;  // workgroups a pair
  // the shared expert's down in the same launch (one token, routed_down_kernel's SHARED form): its Q4_K rows
  // (s_rows x 512 S), its token (512 S float16) and its product out; its unit u (rows 8 u .. 8 u + 7) is taken by
  // wave u % 2 of workgroup u / 2
  const uint8_t* s_blocks;
  const f16* s_x;
  f16* s_out;
  int s_rows, s_row_bytes;
};

// SHARED: the shared expert's down in the same launch, one token. Of a workgroup's sixteen waves, waves 0 and 1
// take a unit of the shared expert's rows each (and no routed unit), waves 2 and 3 two routed units each, and the
// others one: the same sixteen routed units a workgroup, and no wave holds two types' rows (one with both held
// its shared rows' fields through the routed decode and spilled 60 registers). At eight pairs of 4096 rows the
// 256 workgroups take 4096 shared rows: the routed launch alone 8.4 us a layer, with the shared down 8.7-9.1 us,
// the two launches apart 13.2 us.
template <int KIND, int S, int UPW, bool SHARED = false>
__global__ __launch_bounds__(kGluThreads, 4) void routed_down_kernel(DownParams p) {
  typedef Routed<KIND> R;
  typedef Routed<K_Q4_K> RS;
  constexpr int kPairs = 8 * S;        // run pairs of a row
  constexpr int kPieces = 8 * kPairs;  // 16-byte pieces of a token
  static_assert(!SHARED || UPW == 1, "the shared form: sixteen routed units a workgroup");
  __shared__ u32x2 tab[R::kEntries];
  __shared__ u32x4 xs[kPieces];
  __shared__ u32x4 xs2[SHARED ? kPieces : 1];  // the shared expert's token
  const int tid = threadIdx.x, lane = tid & 63, m = lane & 7, sub = lane >> 3;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int pair = blockIdx.x / p.groups_per_pair, chunk = blockIdx.x - pair * p.groups_per_pair;

  // the table entry this thread expands and a piece of the pair's token (and of the shared expert's), asked for first
  const uint64_t entry = R::fetch(tid);
  const u32x4 xpiece = reinterpret_cast<const u32x4*>(p.x + (int64_t)(pair / p.share) * (8 * kPieces))[tid % kPieces];
  u32x4 spiece;
  if constexpr (SHARED) spiece = reinterpret_cast<const u32x4*>(p.s_x)[tid % kPieces];
  const uint32_t e = p.idx[pair];
  const bool bad = e >= p.experts;
  const uint8_t* mat = p.blocks + (int64_t)(bad ? 0u : e) * p.mat_bytes;
  R::fill(tab, tid, entry);
  {
    const int c = tid % kPieces;  // threads past the token's pieces write the same bytes again
    xs[glu_x_slot(c >> 3, c & 7)] = xpiece;
    if constexpr (SHARED) xs2[glu_x_slot(c >> 3, c & 7)] = spiece;
  }
  __syncthreads();

  // N routed units from unit u0 of the pair (rows 8 u0 ..): their rows asked for at once, then each decoded
  auto routed = [&](auto n_units, int u0) {
    constexpr int N = decltype(n_units)::value;
    int r0[N];
#pragma unroll
    for (int k = 0; k < N; ++k) r0[k] = (u0 + k) * 8;  // the unit's first row
    typename R::Fields f[N][S];
#pragma unroll
    for (int k = 0; k < N; ++k) {
      const int rl = min(r0[k] + sub, p.rows - 1);  // rows past the matrix read its last row, and write nothing
      const uint8_t* row = mat + (int64_t)rl * p.row_bytes;
#pragma unroll
      for (int st = 0; st < S; ++st) R::load(row, 8 * st + m, f[k][st]);
      asm volatile("" ::: "memory");
    }
#pragma unroll
    for (int k = 0; k < N; ++k) {
      float acc = 0.0f;
#pragma unroll
      for (int st = 0; st < S; ++st) {
        opaque(f[k][st]);
        const int j = 8 * st + m;
        uint32_t x[32];
#pragma unroll
        for (int v = 0; v < 8; ++v) {
          const u32x4 c = xs[glu_x_slot(j, v)];
#pragma unroll
          for (int i = 0; i < 4; ++i) x[4 * v + i] = c[i];
        }
        float xsum[2 * kXSums<KIND> + 1];
        if constexpr (kBiasedRuns<KIND>) {
          x_sums<KIND>(x, xsum);
          x_sums<KIND>(x + 16, xsum + kXSums<KIND>);
        }
        acc += R::pair_sum_lds(f[k][st], j, x, xsum, tab);
      }
      acc += lanes_apart(acc, 1);
      acc += lanes_apart(acc, 2);
      acc += lanes_apart(acc, 4);
      const int r = r0[k] + sub;
      if (m == 0 && r < p.rows)
        p.out[(int64_t)pair * p.rows + r] = bad ? (f16)__builtin_nanf("") : from_f32<f16>(acc);
    }
  };

  if constexpr (!SHARED) {
    routed(std::integral_constant<int, UPW>(), (chunk * kGluWaves + wave) * UPW);
  } else {
    const int u = chunk * kGluWaves;  // the workgroup's first routed unit
    if (wave >= 4) {
      routed(std::integral_constant<int, 1>(), u + wave);
    } else if (wave >= 2) {
      routed(std::integral_constant<int, 2>(), u + 2 * (wave - 2));
    } else {
      const int s_unit = 2 * blockIdx.x + wave;  // rows 8 s_unit .. of the shared expert's down
      if (8 * s_unit < p.s_rows) {
        typename RS::Fields fs[S];
        const int rl = min(s_unit * 8 + sub, p.s_rows - 1);
        const uint8_t* row = p.s_blocks + (int64_t)rl * p.s_row_bytes;
#pragma unroll
        for (int st = 0; st < S; ++st) RS::load(row, 8 * st + m, fs[st]);
        float acc = 0.0f;
#pragma unroll
        for (int st = 0; st < S; ++st) {
          opaque(fs[st]);
          const int j = 8 * st + m;
          int jx = j;  // read after the last run pair's sum: the token's 32 registers held for one run pair at a time
          asm volatile("" : "+v"(jx) : "v"(acc));
          uint32_t x[32];
#pragma unroll
          for (int v = 0; v < 8; ++v) {
            const u32x4 c = xs2[glu_x_slot(jx, v)];
#pragma unroll
            for (int i = 0; i < 4; ++i) x[4 * v + i] = c[i];
          }
          float xsum[2 * kXSums<K_Q4_K> + 1];
          x_sums<K_Q4_K>(x, xsum);
          x_sums<K_Q4_K>(x + 16, xsum + kXSums<K_Q4_K>);
          acc += RS::pair_sum(fs[st], j, x, xsum, tab);
        }
        acc += lanes_apart(acc, 1);
        acc += lanes_apart(acc, 2);
        acc += lanes_apart(acc, 4);
        const int r = s_unit * 8 + sub;
        if (m == 0 && r < p.s_rows) p.s_out[r] = from_f32<f16>(acc);
      }
    }
  }
}

constexpr bool routed_kind(int kind) { return kind == K_IQ3_S || kind == K_Q2_0; }
constexpr bool routed_linear(int kind) { return kind == K_Q4_K || kind == K_Q6_K || kind == K_Q8_0; }

// Whether routed_down_kernel takes a routed one-matrix call: IQ3_S or Q2_0 rows of 1536 or 2560 inputs, float16
// in and out (the caller has checked the dtypes).
template <int KIND>
bool routed_down_takes(const MatvecParams& p) {
  return routed_kind(KIND) && p.mode == MODE_EXPERT && (p.cols == 1536 || p.cols == 2560) &&
         p.glu_out == nullptr && p.experts <= INT32_MAX && p.pairs <= 65535;
}

template <int KIND, int S, int UPW, bool SHARED = false>
int launch_down_su(DownParams& p, int units_per_pair, hipStream_t s) {
  const int per_group = kGluWaves * UPW;
  p.groups_per_pair = (units_per_pair + per_group - 1) / per_group;
  const int64_t groups = (int64_t)p.groups_per_pair * p.pairs;
  if (groups > INT32_MAX) return STRATA_ERR_SHAPE;
  if (SHARED && (p.s_rows + 7) / 8 > 2 * groups) return STRATA_ERR_SHAPE;  // two shared units a workgroup
  hipLaunchKernelGGL((routed_down_kernel<KIND, S, UPW, SHARED>), dim3((unsigned)groups), dim3(kGluThreads), 0, s, p);
  STRATA_CHECK_LAUNCH();
  return STRATA_OK;
}

template <int KIND>
int launch_routed_down(const MatvecParams& mp, hipStream_t s) {
  if constexpr (!routed_kind(KIND)) {
    return STRATA_ERR_SHAPE;
  } else {
    DownParams p = {};
    p.blocks = mp.blocks[0];
    p.idx = mp.idx;
    p.x = reinterpret_cast<const f16*>(mp.x);
    p.out = reinterpret_cast<f16*>(mp.out[0]);
    p.mat_bytes = mp.mat_bytes;
    p.experts = (uint32_t)mp.experts;
    p.rows = mp.rows;
    p.row_bytes = mp.row_bytes;
    p.pairs = mp.pairs;
    p.share = mp.share;
    const int units_per_pair = (mp.rows + 7) / 8;
    // units a wave, one or two: the fewer rounds of workgroups (a pair's own) times units a wave (40 pairs of
    // 4096 rows: 1280 workgroups of one unit a wave, five full rounds, against 640 of two, two and a half)
    const int64_t cus = (int64_t)device_cus() * kGluGroupsPerCU;
    auto cost = [&](int upw) {
      const int64_t groups = (int64_t)((units_per_pair + kGluWaves * upw - 1) / (kGluWaves * upw)) * mp.pairs;
      return (groups + cus - 1) / cus * upw;
    };
    const bool two = cost(2) < cost(1);
    if (mp.shared[0] != nullptr) {  // the shared expert's down in the launch: rows of 1536 inputs, one unit a wave
      p.s_blocks = mp.shared[0];
      p.s_x = reinterpret_cast<const f16*>(mp.shared_x);
      p.s_out = reinterpret_cast<f16*>(mp.shared_out);
      p.s_rows = mp.shared_rows;
      p.s_row_bytes = mp.shared_row_bytes;
      if (mp.cols != 1536 || two) return STRATA_ERR_SHAPE;
      return launch_down_su<KIND, 3, 1, true>(p, units_per_pair, s);
    }
    if (mp.cols == 1536)
      return two ? launch_down_su<KIND, 3, 2>(p, units_per_pair, s) : launch_down_su<KIND, 3, 1>(p, units_per_pair, s);
    return two ? launch_down_su<KIND, 5, 2>(p, units_per_pair, s) : launch_down_su<KIND, 5, 1>(p, units_per_pair, s);
  }
}

// Whether routed_glu_kernel takes a paired gate/up call: IQ3_S and Q2_0 rows of 4096 inputs at up to eight
// tokens, float16 in and out (the caller has checked the dtypes). The linear types' gate/up (a shared expert's:
// 1536 units, under a round of waves) run 5 % faster on direct_decode_kernel, which spreads them over every CU.
template <int KIND>
bool routed_glu_takes(const MatvecParams& p) {
  const int tokens = p.share > 0 ? p.pairs / p.share : 0;
  return routed_kind(KIND) && tokens <= kGluMaxTokens && p.mode == MODE_EXPERT && p.cols == 4096 &&
         p.glu_out != nullptr && p.experts <= INT32_MAX && (int64_t)p.pairs * p.rows <= INT32_MAX / 2;
}

// Whether routed_glu_kernel's one-matrix form takes a dense matvec: rows of 4096 inputs, one token, every row,
// float16 in and out; Q4_K at 32768 rows or more (an lm_head: 151936 rows in 77 us against 98 us on
// direct_decode_kernel), Q6_K and Q8_0 at up to 16384 (4096 rows: 6.4 against 7.9 us for Q6_K, 6.5 against 8.2 us
// for Q8_0; q, k and v as one 12288-row launch: 13.6 against 14.0 us). Below 32768 rows Q4_K, and above 16384 Q6_K
// (lm_head: 138 against 125 us), run faster on the direct kernel.
template <int KIND>
bool routed_one_takes(const MatvecParams& p) {
  const bool kind = (KIND == K_Q4_K && p.rows >= 32768) || ((KIND == K_Q6_K || KIND == K_Q8_0) && p.rows <= 16384);
  return kind && p.mode == MODE_DENSE && p.cols == 4096 && p.tokens == 1 && p.row_ids == nullptr &&
         p.rows <= INT32_MAX / 2;
}

template <int KIND, int MODE, bool SHARED = false>
int launch_glu_upw(GluParams& p, int upw, dim3 grid, hipStream_t s) {
  const dim3 block(glu_threads<KIND, MODE>());
  switch (upw) {
    case 1: hipLaunchKernelGGL((routed_glu_kernel<KIND, 1, MODE, SHARED>), grid, block, 0, s, p); break;
    case 2: hipLaunchKernelGGL((routed_glu_kernel<KIND, 2, MODE, SHARED>), grid, block, 0, s, p); break;
    case 3: hipLaunchKernelGGL((routed_glu_kernel<KIND, 3, MODE, SHARED>), grid, block, 0, s, p); break;
    case 4: hipLaunchKernelGGL((routed_glu_kernel<KIND, 4, MODE, SHARED>), grid, block, 0, s, p); break;
    case 6: hipLaunchKernelGGL((routed_glu_kernel<KIND, 6, MODE, SHARED>), grid, block, 0, s, p); break;
    case 8: hipLaunchKernelGGL((routed_glu_kernel<KIND, 8, MODE, SHARED>), grid, block, 0, s, p); break;
    case 12: hipLaunchKernelGGL((routed_glu_kernel<KIND, 12, MODE, SHARED>), grid, block, 0, s, p); break;
    case 15: hipLaunchKernelGGL((routed_glu_kernel<KIND, 15, MODE, SHARED>), grid, block, 0, s, p); break;
    case 16: hipLaunchKernelGGL((routed_glu_kernel<KIND, 16, MODE, SHARED>), grid, block, 0, s, p); break;
    case 20:
      if constexpr (MODE == ONE) hipLaunchKernelGGL((routed_glu_kernel<KIND, 20, MODE, SHARED>), grid, block, 0, s, p);
      break;
    default: hipLaunchKernelGGL((routed_glu_kernel<KIND, 24, MODE, SHARED>), grid, block, 0, s, p); break;
  }
  STRATA_CHECK_LAUNCH();
  return STRATA_OK;
}

// Units a wave: the fewest of the forms built that fit the units into one round of resident waves (IQ3_S at two,
// eight, 15 and 24 units spills registers: three, twelve and 16 instead); at most 24, more waves beyond.
template <int KIND, int MODE>
int glu_units_a_wave(int64_t units) {
  const int64_t capacity = (int64_t)device_cus() * kGluGroupsPerCU * (glu_threads<KIND, MODE>() / 64);
  const int64_t need = (units + capacity - 1) / capacity;
  // 15: five tokens' 40 pairs on every CU; 20 (one-matrix form only): a Q4_K lm_head's 75968 units of two rows
  // in 238 workgroups (at 24, 198 of the 256 CUs: 74 against 68 us)
  static const int kForms[] = {1, 2, 3, 4, 6, 8, 12, 15, 16, 20, 24};
  for (int f : kForms) {
    if (KIND == K_IQ3_S && (f == 2 || f == 8 || f == 15 || f == 24)) continue;
    if (MODE != ONE && f == 20) continue;
    if (f >= need) return f;
  }
  return KIND == K_IQ3_S ? 16 : 24;
}

template <int KIND, int MODE, bool SHARED = false>
int launch_glu_mode(GluParams& p, hipStream_t s) {
  const int64_t units = (int64_t)p.na * p.nb;
  const int upw = glu_units_a_wave<KIND, MODE>(units);
  constexpr int kWaves = glu_threads<KIND, MODE>() / 64;
  const int64_t waves = ((units + upw - 1) / upw + kWaves - 1) / kWaves * kWaves;
  if (waves > INT32_MAX) return STRATA_ERR_SHAPE;
  p.waves = (int)waves;
  p.wave_a = p.waves / p.nb;
  p.wave_b = p.waves % p.nb;
  // one shared unit a wave at most; above 12 units a wave the shared unit's rows spill registers
  if (SHARED && (p.s_rows > p.waves || upw > 12)) return STRATA_ERR_SHAPE;
  return launch_glu_upw<KIND, MODE, SHARED>(p, upw, dim3((unsigned)(waves / kWaves)), s);
}

// The ROUTE form: the one-token shared form at three units a wave (eight pairs of 1536 rows), the choice of experts
// in the launch; other shapes return STRATA_ERR_SHAPE (the router's choice then comes from its own launch).
template <int KIND>
int launch_glu_route(GluParams& p, hipStream_t s) {
  const int64_t units = (int64_t)p.na * p.nb;
  constexpr int kWaves = glu_threads<KIND, GLU1>() / 64;
  if (glu_units_a_wave<KIND, GLU1>(units) != 3 || p.pairs > 64 || p.r_experts > 256 || p.r_experts < p.pairs ||
      p.r_rows < p.r_experts)
    return STRATA_ERR_SHAPE;
  const int64_t waves = ((units + 2) / 3 + kWaves - 1) / kWaves * kWaves;
  p.waves = (int)waves;
  p.wave_a = p.waves / p.nb;
  p.wave_b = p.waves % p.nb;
  if (p.s_rows > p.waves) return STRATA_ERR_SHAPE;  // one shared unit a wave at most
  hipLaunchKernelGGL((routed_glu_kernel<KIND, 3, GLU1, true, true>), dim3((unsigned)(waves / kWaves)),
                     dim3(glu_threads<KIND, GLU1>()), 0, s, p);
  STRATA_CHECK_LAUNCH();
  return STRATA_OK;
}

template <int KIND>
int launch_routed_glu(const MatvecParams& mp, hipStream_t s) {
  if constexpr (!routed_kind(KIND)) {
    return STRATA_ERR_SHAPE;
  } else {
    GluParams p = {};
    p.gate = mp.blocks[0];
    p.up = mp.blocks[1];
    p.idx = mp.idx;
    p.x = reinterpret_cast<const u32x4*>(mp.x);
    p.out_gate = reinterpret_cast<f16*>(mp.out[0]);
    p.out_up = reinterpret_cast<f16*>(mp.out[1]);
    p.h = reinterpret_cast<f16*>(mp.glu_out);
    p.mat_bytes = mp.mat_bytes;
    p.experts = (uint32_t)mp.experts;
    p.rows = mp.rows;
    p.row_bytes = mp.row_bytes;
    p.pairs = mp.pairs;
    p.share = mp.share;
    p.tokens = mp.pairs / mp.share;
    if (mp.shared[0] != nullptr) {  // the shared expert's gate and up in the same launch: one token
      if (p.tokens != 1 || mp.shared_rows < 1) return STRATA_ERR_SHAPE;
      if (mp.route_logits != nullptr) {  // and the choice of experts
        p.r_logits = mp.route_logits;
        p.r_idx = mp.route_idx;
        p.r_w = mp.route_w;
        p.r_extra = reinterpret_cast<f16*>(mp.route_extra);
        p.r_rows = mp.route_rows;
        p.r_experts = mp.route_experts;
      }
      p.s_gate = mp.shared[0];
      p.s_up = mp.shared[1];
      p.s_h = reinterpret_cast<f16*>(mp.shared_out);
      p.s_g = reinterpret_cast<f16*>(mp.shared_gu[0]);
      p.s_u = reinterpret_cast<f16*>(mp.shared_gu[1]);
      p.s_rows = mp.shared_rows;
      p.s_row_bytes = mp.shared_row_bytes;
      p.na = p.pairs;
      p.nb = p.rows;
      if (mp.route_logits != nullptr) return launch_glu_route<KIND>(p, s);
      return launch_glu_mode<KIND, GLU1, true>(p, s);
    }
    if (p.tokens > 1) {
      p.na = p.pairs;
      p.nb = p.rows;
      return launch_glu_mode<KIND, GLUN>(p, s);
    }
    p.na = p.pairs;
    p.nb = p.rows;
    return launch_glu_mode<KIND, GLU1>(p, s);
  }
}

// Whether the float32 form (ONE32) takes a dense matvec: Q4_K rows of 4096 inputs, one float32 token, float32
// out, every row.
template <int KIND>
bool routed_one32_takes(const MatvecParams& p) {
  return KIND == K_Q4_K && p.mode == MODE_DENSE && p.cols == 4096 && p.tokens == 1 && p.row_ids == nullptr &&
         p.rows <= INT32_MAX / 2;
}

template <int KIND, bool F32 = false>
int launch_routed_one(const MatvecParams& mp, hipStream_t s) {
  if constexpr ((KIND != K_Q4_K && KIND != K_Q6_K && KIND != K_Q8_0) || (F32 && KIND != K_Q4_K)) {
    return STRATA_ERR_SHAPE;
  } else {
    GluParams p = {};
    p.gate = mp.blocks[0];
    p.x = reinterpret_cast<const u32x4*>(mp.x);
    p.out_gate = reinterpret_cast<f16*>(mp.out[0]);
    p.row_bytes = mp.row_bytes;
    p.rows = mp.rows;
    p.pairs = 1;
    p.share = 1;
    p.tokens = 1;
    p.na = 1;
    p.nb = (mp.rows + 1) / 2;
    return F32 ? launch_glu_mode<KIND, ONE32>(p, s) : launch_glu_mode<KIND, ONE>(p, s);
  }
}

}  // namespace strata_mv
