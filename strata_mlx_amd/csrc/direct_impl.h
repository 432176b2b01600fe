// The decode matvec for float16 activations, rows read straight into registers (IQ3_S, IQ3_XXS, Q2_0 with
// their codebooks in LDS; Q3_K, Q4_K, Q6_K, Q8_0, Q4_0, Q5_0 decoded by byte arithmetic; IQ4_XS, IQ4_NL through
// an LDS table of codebook pairs).
//
// A decode call moves tens of megabytes in a few microseconds, so what matters is that every byte is requested
// at once: a wave's loads go out as soon as it knows its expert, before anything else it does. Nothing is staged
// in LDS except the codebooks and a token the workgroup shares. A lane takes two consecutive runs of one block
// (64 weights) of a row and loads exactly their fields into registers (IQ3_S: the 16 index bytes, the two
// high-bit bytes, the eight sign bytes, the scale bytes and d: five loads at 2-byte alignment, which gfx950 serves
// as they are). A row is L lanes (its run pairs rounded up to a power of two: 64 for 4096 inputs, 32 for 1536),
// 64 / L rows side by side; a wave takes RU such row steps of one matrix (a "unit"), all loaded before the first
// is decoded, and decodes each step as soon as that step's own loads are in. Codebook entries come from LDS as
// float16 and sign masks, products from v_dot2_f32_f16 against the activations packed in registers, and a row's
// partial sums meet across its lanes by DPP and row swaps. Rows of 24 or 40 run pairs, which fill such rows
// badly, take direct_odd_kernel: 8 lanes a row, every lane busy.
//
// The routed form gives a wave (pair, stack, rows), from a grid of (units, stacks, pairs). A pair whose expert
// an earlier pair names leaves its rows to that pair's waves, which multiply them by every pair naming the expert
// (ballots over the pairs' ids, TT pairs a pass). When every pair multiplies the same token (one token's
// gate/up), the rows are multiplied once and the sum is written for every pair naming the expert.
//
// Paired mode (gate and up of one call): a unit's row steps alternate between the two stacks, the same rows of
// each, so the lane that ends with row r's gate sum also has its up sum, and writes silu(gate) * up as mlx-lm
// rounds it (strata_mlx/blocks.py:222-236): the down projection then reads one float16 vector a pair.
#pragma once
#include "decode_impl.h"

namespace strata_mv {

constexpr int kDMaxPairs = 256;  // pairs the direct kernel takes (four ballots)
constexpr int kDMaxCols = 4096;  // inputs of a row the direct kernel takes (64 lanes of 64)
constexpr int kDMaxGridY = 65535;  // pairs (and stacks) of a launch: the grid's y and z

// the fields of two consecutive runs of a block, as one lane holds them
template <int KIND>
struct RunPair;
template <>
struct RunPair<K_IQ3_S> {
  u32x4 qs;     // 16 index bytes
  uint16_t qh;  // two high-bit bytes
  u32x2 sg;     // eight sign bytes
  uint16_t sc;  // the block's scale bytes 2 (j % 4 / 2), + 1: byte j % 2 the lane's (low nibble run 2j's)
  uint16_t d;
};
template <>
struct RunPair<K_IQ3_XXS> {
  u32x4 qs;
  u32x2 aux;    // the two runs' scale and sign words
  uint16_t d;
};
template <>
struct RunPair<K_Q2_0> {
  u32x4 qs;     // the block's 16 code bytes
  uint16_t d;
};
// The kinds decoded without a codebook: a lane's 64 weights are two Q8_0 blocks, a quarter of a Q4_K block (the
// low and high nibbles of 32 bytes), or two runs of a Q6_K half block (r0 and r0 + 2: the low and high nibbles of
// 32 ql bytes, bits 2r .. 2r + 1 of the half's 32 qh bytes).
template <>
struct RunPair<K_Q8_0> {
  u32x4 q[4];   // the two blocks' 32 int8 codes each
  uint16_t d[2];
};
template <>
struct RunPair<K_Q4_K> {
  u32x4 qs[2];  // 32 bytes: the first run's codes in the low nibbles, the second's in the high
  u32x4 sm;     // the 12 packed scale / min bytes (and 4 bytes past them)
  uint32_t dd;  // d | dmin << 16
};
template <>
struct RunPair<K_Q6_K> {
  u32x4 ql[2];     // 32 bytes: run r0's low four bits in the low nibbles, run r0 + 2's in the high
  u32x4 qh[2];     // the half's 32 high-bit bytes
  uint16_t sc[2];  // each run's two int8 scales (16 weights a scale)
  uint16_t d;
};

template <>
struct RunPair<K_Q3_K> {
  u32x4 qs[2];   // the 32 code bytes of the lane's two runs (2 bits a weight, run 2jj + h at bit 4 (jj % 2) + 2h)
  u32x4 hm[2];   // the 32 high-bit bytes (run r at bit r)
  uint32_t lo;   // the low four bits of the lane's four 6-bit scales (at bit 4 (jj / 2) of each byte)
  uint32_t hi;   // their high two bits (at bit 2 jj of each byte)
  uint16_t d;
};

template <>
struct RunPair<K_IQ4_XS> {
  u32x4 qs[2];   // the lane's two runs' 16 code bytes each (weights 0-15 in the low nibbles, 16-31 in the high)
  uint32_t dh;   // d | scales_h << 16
  uint32_t sl;   // the four scales_l bytes (run 2k's low four scale bits in byte k's low nibble)
};

template <>
struct RunPair<K_IQ4_NL> {
  u32x4 qs[2];     // the lane's two blocks' 16 code bytes each
  uint16_t d[2];
};

template <>
struct RunPair<K_Q5_K> {
  u32x4 qs[2];  // as Q4_K's
  u32x4 qh[2];  // the block's 32 high-bit bytes (sub-block s at bit s)
  u32x4 sm;
  uint32_t dd;
};

// Q4_0 and Q5_0: two blocks of 32 weights a lane (Q5_0: their high bits in a word each)
template <>
struct RunPair<K_Q4_0> {
  u32x4 qs[2];
  uint16_t d[2];
};
template <>
struct RunPair<K_Q5_0> {
  u32x4 qs[2];
  uint32_t qh[2];
  uint16_t d[2];
};

template <int KIND>
struct DirectKind {
  static constexpr bool linear = KIND == K_Q8_0 || KIND == K_Q4_K || KIND == K_Q5_K || KIND == K_Q6_K ||
                                 KIND == K_Q3_K || KIND == K_IQ4_XS || KIND == K_IQ4_NL || KIND == K_Q4_0 ||
                                 KIND == K_Q5_0;
  static constexpr bool any = FastTraits<KIND>::supported || linear;
  // a table of two codebook values a byte (the 16-entry IQ4 codebook)
  static constexpr int pair_codes = KIND == K_IQ4_XS || KIND == K_IQ4_NL ? 256 : 0;
};

// A load from global memory at any alignment (gfx950 serves 2-byte aligned dwordx2/x4 loads as they are).
template <typename T>
struct __attribute__((packed, aligned(1))) Unaligned {
  T v;
};
template <typename T>
__device__ __forceinline__ T load_unaligned(const uint8_t* p) {
  typedef const __attribute__((address_space(1))) Unaligned<T> GlobalT;
  return ((GlobalT*)(const __attribute__((address_space(1))) uint8_t*)p)->v;
}

__device__ __forceinline__ float half_bits(uint32_t b) { return (float)__builtin_bit_cast(f16, (uint16_t)b); }

// The LDS tables of the register decode: codebook entries as four float16 integers, and the XOR masks of four
// sign bits (16 entries of 8 bytes: one row of banks, so lanes reading different entries never conflict).
template <int KIND>
struct DirectTables {
  u32x2 grid[FastTraits<KIND>::grid > 0 ? FastTraits<KIND>::grid : 1];
  u32x2 sign4[16];
  u32x2 q2[FastTraits<KIND>::q2 > 0 ? FastTraits<KIND>::q2 : 1];  // a Q2_0 code byte: four (c - 1)
  // IQ4_XS / IQ4_NL: byte lo | hi << 4 -> the float16 pair (kvalues[lo], kvalues[hi])
  uint32_t kv2[DirectKind<KIND>::pair_codes > 0 ? DirectKind<KIND>::pair_codes : 1];
};

// (byte K of v) << sh and (16-bit word K of v) << sh in one instruction each: a shift whose operand is a byte /
// word select (SDWA). The compiler selects these forms itself for the upper bytes and word, and two
// instructions (shift, mask) for the lowest. sh is a register (3: table entries of 8 bytes, 2: of 4).
template <int K>
__device__ __forceinline__ uint32_t byte_shl(uint32_t v, uint32_t three) {
  uint32_t r;
  if constexpr (K == 0)
    asm("v_lshlrev_b32_sdwa %0, %1, %2 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_0"
        : "=v"(r) : "v"(three), "v"(v));
  else if constexpr (K == 1)
    asm("v_lshlrev_b32_sdwa %0, %1, %2 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_1"
        : "=v"(r) : "v"(three), "v"(v));
  else if constexpr (K == 2)
    asm("v_lshlrev_b32_sdwa %0, %1, %2 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_2"
        : "=v"(r) : "v"(three), "v"(v));
  else
    asm("v_lshlrev_b32_sdwa %0, %1, %2 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_3"
        : "=v"(r) : "v"(three), "v"(v));
  return r;
}
template <int K>
__device__ __forceinline__ uint32_t word_shl(uint32_t v, uint32_t three) {
  uint32_t r;
  if constexpr (K == 0)
    asm("v_lshlrev_b32_sdwa %0, %1, %2 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:WORD_0"
        : "=v"(r) : "v"(three), "v"(v));
  else
    asm("v_lshlrev_b32_sdwa %0, %1, %2 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:WORD_1"
        : "=v"(r) : "v"(three), "v"(v));
  return r;
}

// 8 bytes of LDS at byte offset off from table t
__device__ __forceinline__ u32x2 lds_entry(const u32x2* t, uint32_t off) {
  return *reinterpret_cast<const u32x2*>(reinterpret_cast<const char*>(t) + off);
}

// run h (0, 1) of a pair: 16 packed float16 pairs of integers, and the run's scale
template <int KIND>
__device__ __forceinline__ float decode_pair(const RunPair<KIND>& f, int h, int j, uint32_t* w,
                                             const DirectTables<KIND>& t) {
  const float d = half_bits(f.d);
  if constexpr (KIND == K_IQ3_S) {  // strata_mlx/blocks.py:89-102
    const uint32_t qs0 = f.qs[2 * h], qs1 = f.qs[2 * h + 1];
    const uint32_t qh = (f.qh >> (8 * h)) & 255, sg = f.sg[h];
    const float scale = d * (float)(1 + 2 * __builtin_amdgcn_ubfe((uint32_t)f.sc, 8 * (j & 1) + 4 * h, 4));
    // the ninth index bits of four groups spread into bytes, then interleaved with the qs bytes by v_perm
    const uint32_t hb0 = (__builtin_amdgcn_ubfe(qh, 0, 4) * 0x204081u) & 0x01010101u;
    const uint32_t hb1 = (__builtin_amdgcn_ubfe(qh, 4, 4) * 0x204081u) & 0x01010101u;
    const uint32_t i01 = __builtin_amdgcn_perm(hb0, qs0, 0x05010400u), i23 = __builtin_amdgcn_perm(hb0, qs0, 0x07030602u);
    const uint32_t i45 = __builtin_amdgcn_perm(hb1, qs1, 0x05010400u), i67 = __builtin_amdgcn_perm(hb1, qs1, 0x07030602u);
    const uint32_t three = 3;
    // byte offsets of the codebook entries (index * 8) and of the sign masks (nibble * 8): the sign nibbles split
    // into the bytes of two words (groups 0, 2, 4, 6 and 1, 3, 5, 7), each then one byte select
    const uint32_t ga[8] = {word_shl<0>(i01, three), word_shl<1>(i01, three), word_shl<0>(i23, three),
                            word_shl<1>(i23, three), word_shl<0>(i45, three), word_shl<1>(i45, three),
                            word_shl<0>(i67, three), word_shl<1>(i67, three)};
    const uint32_t se = sg & 0x0F0F0F0Fu, so = (sg >> 4) & 0x0F0F0F0Fu;
    const uint32_t sa[8] = {byte_shl<0>(se, three), byte_shl<0>(so, three), byte_shl<1>(se, three),
                            byte_shl<1>(so, three), byte_shl<2>(se, three), byte_shl<2>(so, three),
                            byte_shl<3>(se, three), byte_shl<3>(so, three)};
#pragma unroll
    for (int l = 0; l < 8; ++l) {
      const u32x2 g = lds_entry(t.grid, ga[l]);
      const u32x2 m = lds_entry(t.sign4, sa[l]);
      w[2 * l] = g[0] ^ m[0];
      w[2 * l + 1] = g[1] ^ m[1];
    }
    return scale;
  } else if constexpr (KIND == K_IQ3_XXS) {  // strata_mlx/blocks.py:103-116
    const uint32_t qs0 = f.qs[2 * h], qs1 = f.qs[2 * h + 1];
    const uint32_t aux = f.aux[h];
    const float scale = d * (0.5f + (float)(aux >> 28)) * 0.5f;
#pragma unroll
    for (int l = 0; l < 8; ++l) {
      const u32x2 g = t.grid[((l < 4 ? qs0 : qs1) >> (8 * (l & 3))) & 255];
      const uint32_t s7 = (aux >> (7 * (l >> 1))) & 127;
      // ksigns: the parity in bit 7 (the count's bit 0; its bits 1-2 land in bits 8-9, which the nibbles leave out)
      const uint32_t s8 = s7 | ((uint32_t)__builtin_popcount(s7) << 7);
      const u32x2 m = t.sign4[(s8 >> (4 * (l & 1))) & 15];
      w[2 * l] = g[0] ^ m[0];
      w[2 * l + 1] = g[1] ^ m[1];
    }
    return scale;
  } else {  // Q2_0, strata_mlx/blocks.py:58-68
    const uint32_t q0 = f.qs[2 * h], q1 = f.qs[2 * h + 1];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const u32x2 c = t.q2[((i < 4 ? q0 : q1) >> (8 * (i & 3))) & 255];
      w[2 * i] = c[0];
      w[2 * i + 1] = c[1];
    }
    return d;
  }
}

// Four code bytes -> two words of float16 integers, each code less `bias`: 0x64nn is 1024 + nn, and 1024 + bias
// is subtracted from both halves at once (exact: integers below 2048).
template <int BIAS>
__device__ __forceinline__ void bytes_to_h2(uint32_t b, uint32_t* w2) {
  typedef _Float16 h2v __attribute__((ext_vector_type(2)));
  const h2v k = h2v{(_Float16)(1024.0f + BIAS), (_Float16)(1024.0f + BIAS)};
  w2[0] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2v, __builtin_amdgcn_perm(0x64646464u, b, 0x04010400u)) - k);
  w2[1] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2v, __builtin_amdgcn_perm(0x64646464u, b, 0x04030402u)) - k);
}

// Four code bytes -> two words of float16 1024 + code (exact), the bias left to the sum: 1024 + code times x
// summed is the codes' sum plus 1024 times the sum of x, which apply_run takes off once a run (or half run), not
// once a weight pair.
__device__ __forceinline__ void bytes_to_h2_biased(uint32_t b, uint32_t* w2) {
  w2[0] = __builtin_amdgcn_perm(0x64646464u, b, 0x04010400u);
  w2[1] = __builtin_amdgcn_perm(0x64646464u, b, 0x04030402u);
}
// The kinds whose decode_run leaves that bias in: the sum of x it needs (x_sums) is the lane's, the same for
// every row, so the matvecs compute it once a token.
template <int KIND>
constexpr bool kBiasedRuns = KIND == K_Q4_K || KIND == K_Q5_K || KIND == K_Q6_K;

// A run's scales: a (every kind), b (Q4_K: dmin * min, subtracted times the run's sum of x; Q6_K: the second
// 16 weights' scale, a the first 16's).
struct RunScale {
  float a, b;
};

// A run's 16 code bytes of the IQ4 codebook -> its 32 weights as 16 float16 pairs, from the pair table kv2.
// Four code bytes b0..b3: their low nibbles are weights 4k .. 4k + 3, their high ones 16 + 4k ..; OR-ing the
// nibbles with themselves four bits down puts the pairs (b0, b1) and (b2, b3) in bytes 0 and 2: the index of
// the pair table, two weights a lookup.
__device__ __forceinline__ void pair_codes_run(const u32x4& qs, uint32_t* w, const uint32_t* kv2) {
  const uint32_t two = 2;
  const char* base = reinterpret_cast<const char*>(kv2);
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const uint32_t q = qs[k];
    const uint32_t lo = q & 0x0F0F0F0Fu, hi = (q >> 4) & 0x0F0F0F0Fu;
    const uint32_t tl = lo | (lo >> 4), th = hi | (hi >> 4);
    w[2 * k] = *reinterpret_cast<const uint32_t*>(base + byte_shl<0>(tl, two));
    w[2 * k + 1] = *reinterpret_cast<const uint32_t*>(base + byte_shl<2>(tl, two));
    w[8 + 2 * k] = *reinterpret_cast<const uint32_t*>(base + byte_shl<0>(th, two));
    w[9 + 2 * k] = *reinterpret_cast<const uint32_t*>(base + byte_shl<2>(th, two));
  }
}

// Run h (0, 1) of lane run pair j: 16 packed float16 pairs of integers into w, and its scales.
template <int KIND>
__device__ __forceinline__ RunScale decode_run(const RunPair<KIND>& f, int h, int j, uint32_t* w,
                                               const DirectTables<KIND>& t) {
  if constexpr (KIND == K_Q8_0) {  // w = d * q, strata_mlx/gguf.py:203-206
#pragma unroll
    for (int i = 0; i < 8; ++i) bytes_to_h2<128>(f.q[2 * h + i / 4][i % 4] ^ 0x80808080u, w + 2 * i);
    return RunScale{half_bits(f.d[h]), 0.0f};
  } else if constexpr (KIND == K_Q4_K || KIND == K_Q5_K) {
    // w = code * (d * sc) - dmin * mn, strata_mlx/gguf.py:174-179, 207-218; Q5_K's codes take bit s of the
    // high-bit bytes as their fifth bit
    const int sb = 2 * (j & 3) + h, tb = 8 * (sb & 3);  // sub-block s of the block
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      uint32_t c = (f.qs[i / 4][i % 4] >> (4 * h)) & 0x0F0F0F0Fu;
      if constexpr (KIND == K_Q5_K) c |= ((f.qh[i / 4][i % 4] >> sb) & 0x01010101u) << 4;
      bytes_to_h2_biased(c, w + 2 * i);  // 1024 + code
    }
    // its 6-bit scale and min from the 12 packed bytes p
    const uint32_t b0 = (f.sm[0] >> tb) & 255, b1 = (f.sm[1] >> tb) & 255, b2 = (f.sm[2] >> tb) & 255;
    const bool hi = sb >= 4;
    const uint32_t sc = hi ? ((b2 & 15) | ((b0 >> 6) << 4)) : (b0 & 63);
    const uint32_t mn = hi ? ((b2 >> 4) | ((b1 >> 6) << 4)) : (b1 & 63);
    return RunScale{half_bits(f.dd & 0xffff) * (float)sc, half_bits(f.dd >> 16) * (float)mn};
  } else if constexpr (KIND == K_Q6_K) {  // w = (code - 32) * scale * d, strata_mlx/gguf.py:150-165
    const int r2 = 2 * ((j & 1) + 2 * h);  // the run's bits in the high-bit bytes
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t lo = (f.ql[i / 4][i % 4] >> (4 * h)) & 0x0F0F0F0Fu;
      const uint32_t hb = (f.qh[i / 4][i % 4] >> r2) & 0x03030303u;
      bytes_to_h2_biased(lo | (hb << 4), w + 2 * i);  // 1024 + code: 1056 + the weight's (code - 32)
    }
    const float d = half_bits(f.d);
    return RunScale{d * (float)(int8_t)(f.sc[h] & 255), d * (float)(int8_t)(f.sc[h] >> 8)};
  } else if constexpr (KIND == K_Q3_K) {  // w = (q - (hmask bit ? 0 : 4)) * (scale - 32) * d, strata_mlx/blocks.py:164-175
    const int jj = j & 3, r = 2 * jj + h;  // the block's run
    const int qsh = 4 * (jj & 1) + 2 * h;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t q = (f.qs[i / 4][i % 4] >> qsh) & 0x03030303u;
      const uint32_t m = (f.hm[i / 4][i % 4] >> r) & 0x01010101u;
      bytes_to_h2<4>(q | (m << 2), w + 2 * i);
    }
    // 6-bit scales 2r and 2r + 1 of the block (strata_mlx/blocks.py:49-53): byte p = 2h, 2h + 1 of the lane's words
    const float d = half_bits(f.d);
    float sc[2];
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const int p = 2 * h + e;
      const uint32_t v = ((f.lo >> (8 * p + 4 * (jj >> 1))) & 15) | (((f.hi >> (8 * p + 2 * jj)) & 3) << 4);
      sc[e] = d * (float)((int)v - 32);
    }
    return RunScale{sc[0], sc[1]};
  } else if constexpr (KIND == K_Q4_0) {  // w = d * (code - 8), strata_mlx/gguf.py:195-197
#pragma unroll
    for (int k = 0; k < 4; ++k) {  // byte i's low nibble is weight i, its high nibble weight 16 + i
      bytes_to_h2<8>(f.qs[h][k] & 0x0F0F0F0Fu, w + 2 * k);
      bytes_to_h2<8>((f.qs[h][k] >> 4) & 0x0F0F0F0Fu, w + 8 + 2 * k);
    }
    return RunScale{half_bits(f.d[h]), 0.0f};
  } else if constexpr (KIND == K_Q5_0) {  // w = d * ((code | high bit << 4) - 16), strata_mlx/gguf.py:198-202
    const uint32_t qh = f.qh[h];
#pragma unroll
    for (int k = 0; k < 4; ++k) {  // weight i's high bit is bit i of qh: four of them spread to bit 4 of bytes
      const uint32_t hl = ((__builtin_amdgcn_ubfe(qh, 4 * k, 4) * 0x204081u) & 0x01010101u) << 4;
      const uint32_t hh = ((__builtin_amdgcn_ubfe(qh, 16 + 4 * k, 4) * 0x204081u) & 0x01010101u) << 4;
      bytes_to_h2<16>((f.qs[h][k] & 0x0F0F0F0Fu) | hl, w + 2 * k);
      bytes_to_h2<16>(((f.qs[h][k] >> 4) & 0x0F0F0F0Fu) | hh, w + 8 + 2 * k);
    }
    return RunScale{half_bits(f.d[h]), 0.0f};
  } else if constexpr (KIND == K_IQ4_NL) {  // w = d * kvalues[code], strata_mlx/blocks.py:69-77
    pair_codes_run(f.qs[h], w, t.kv2);
    return RunScale{half_bits(f.d[h]), 0.0f};
  } else if constexpr (KIND == K_IQ4_XS) {  // w = d * (ls - 32) * kvalues[code], strata_mlx/blocks.py:78-88
    pair_codes_run(f.qs[h], w, t.kv2);
    const int jj = j & 3, ib = 2 * jj + h;  // the block's run
    const uint32_t ls = ((f.sl >> (8 * jj + 4 * h)) & 15) | (((f.dh >> (16 + 2 * ib)) & 3) << 4);
    return RunScale{half_bits(f.dh & 0xffff) * (float)((int)ls - 32), 0.0f};
  } else {
    return RunScale{decode_pair<KIND>(f, h, j, w, t), 0.0f};
  }
}

// Sum of 2n packed float16 products, in two float32 chains (as dot16x2 adds them).
template <int N>
__device__ __forceinline__ float dot_n(const uint32_t* w, const uint32_t* x) {
  float a = 0.0f, b = 0.0f;
#pragma unroll
  for (int i = 0; i < N; i += 2) {
    a = __builtin_amdgcn_fdot2(__builtin_bit_cast(h2_t, w[i]), __builtin_bit_cast(h2_t, x[i]), a, false);
    b = __builtin_amdgcn_fdot2(__builtin_bit_cast(h2_t, w[i + 1]), __builtin_bit_cast(h2_t, x[i + 1]), b, false);
  }
  return a + b;
}

// The sums of x a biased run needs (kBiasedRuns): Q4_K, Q5_K the run's 32 activations; Q6_K each half's 16.
template <int KIND>
__device__ __forceinline__ void x_sums(const uint32_t* x, float* xs) {
  const uint32_t ones[16] = {0x3C003C00u, 0x3C003C00u, 0x3C003C00u, 0x3C003C00u, 0x3C003C00u, 0x3C003C00u,
                             0x3C003C00u, 0x3C003C00u, 0x3C003C00u, 0x3C003C00u, 0x3C003C00u, 0x3C003C00u,
                             0x3C003C00u, 0x3C003C00u, 0x3C003C00u, 0x3C003C00u};
  if constexpr (KIND == K_Q6_K) {
    xs[0] = dot_n<8>(ones, x);
    xs[1] = dot_n<8>(ones, x + 8);
  } else if constexpr (KIND == K_Q4_K || KIND == K_Q5_K) {
    xs[0] = dot_n<16>(ones, x);
  }
}
// per run h of a lane's run pair: the floats of x_sums at xs + kXSums * h
template <int KIND>
constexpr int kXSums = KIND == K_Q6_K ? 2 : kBiasedRuns<KIND> ? 1 : 0;

// The run's sum against 32 activations (16 packed pairs); xs: the run's sums of x (x_sums) for a biased run.
template <int KIND>
__device__ __forceinline__ float apply_run(const RunScale& s, const uint32_t* w, const uint32_t* x, const float* xs) {
  if constexpr (KIND == K_Q4_K || KIND == K_Q5_K) {  // a (code . x) - b sum x, the codes 1024 too high
    return s.a * dot16x2(w, x) - (s.b + 1024.0f * s.a) * xs[0];
  } else if constexpr (KIND == K_Q6_K) {  // a scale every 16 weights, the weights 1056 too high
    return s.a * (dot_n<8>(w, x) - 1056.0f * xs[0]) + s.b * (dot_n<8>(w + 8, x + 8) - 1056.0f * xs[1]);
  } else if constexpr (KIND == K_Q3_K) {  // a scale every 16 weights
    return s.a * dot_n<8>(w, x) + s.b * dot_n<8>(w + 8, x + 8);
  } else {
    return s.a * dot16x2(w, x);
  }
}
// the same with the sums of x taken here
template <int KIND>
__device__ __forceinline__ float apply_run(const RunScale& s, const uint32_t* w, const uint32_t* x) {
  float xs[2] = {0.0f, 0.0f};
  if constexpr (kBiasedRuns<KIND>) x_sums<KIND>(x, xs);
  return apply_run<KIND>(s, w, x, xs);
}

// float16 bits of a non-negative integer below 2048 (exact): the codebooks' float16 entries, at compile time.
constexpr uint32_t f16_bits_of(uint32_t n) {
  if (n == 0) return 0;
  int e = 0;
  while ((n >> (e + 1)) != 0) ++e;  // floor(log2 n)
  return ((uint32_t)(e + 15) << 10) | ((n << (10 - e)) & 0x3FFu);
}
template <int N>
struct HalfGrid {
  uint64_t v[N];  // entry i's four bytes as float16, the first in the low 16 bits
};
template <int N>
constexpr HalfGrid<N> half_grid(const uint32_t (&g)[N]) {
  HalfGrid<N> r{};
  for (int i = 0; i < N; ++i) {
    const uint64_t lo = f16_bits_of(g[i] & 255) | (f16_bits_of((g[i] >> 8) & 255) << 16);
    const uint64_t hi = f16_bits_of((g[i] >> 16) & 255) | (f16_bits_of(g[i] >> 24) << 16);
    r.v[i] = lo | (hi << 32);
  }
  return r;
}
static constexpr HalfGrid<512> kIq3sHalfGrid = half_grid(kStrataIq3sGrid);
static constexpr HalfGrid<256> kIq3xxsHalfGrid = half_grid(kStrataIq3xxsGrid);

// float16 bits of a small signed integer (|n| < 2048)
constexpr uint32_t f16_bits_signed(int n) { return n < 0 ? 0x8000u | f16_bits_of((uint32_t)-n) : f16_bits_of(n); }
// An IQ4 code byte lo | hi << 4 -> (kvalues[lo], kvalues[hi]) as float16. (Q2_0's table of four (c - 1) is
// computed in registers instead: loaded, it puts a memory latency ahead of the workgroup barrier, 8 % slower.)
struct PairCodes {
  uint32_t v[256];
};
constexpr PairCodes pair_codes() {
  PairCodes t{};
  for (int i = 0; i < 256; ++i)
    t.v[i] = f16_bits_signed(kStrataKvaluesIq4nl[i & 15]) | (f16_bits_signed(kStrataKvaluesIq4nl[i >> 4]) << 16);
  return t;
}
static constexpr PairCodes kPairCodes = pair_codes();

// The codebook tables in two halves: the constants' loads go out before the rows' (a wait for them is then not
// a wait for the rows), the LDS entries are written after. The entries are loaded as float16 already.
template <int KIND>
struct TableFetch {
  uint64_t g[2] = {0, 0};  // codebook entries
  uint32_t b = 0;          // IQ4: the pair table's entry
};
template <int KIND, int NT = kThreads>  // NT threads to the workgroup
__device__ __forceinline__ void fetch_tables(TableFetch<KIND>& tf, int tid) {
  if constexpr (FastTraits<KIND>::grid > 0) {
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const int i = min(tid + k * NT, FastTraits<KIND>::grid - 1);
      tf.g[k] = KIND == K_IQ3_S ? kIq3sHalfGrid.v[i] : kIq3xxsHalfGrid.v[i];
    }
  }
  static_assert(NT >= 256, "one pair-table entry a thread");
  if constexpr (DirectKind<KIND>::pair_codes > 0) tf.b = kPairCodes.v[min(tid, 255)];
}
template <int KIND, int NT = kThreads>
__device__ __forceinline__ void store_tables(DirectTables<KIND>& t, const TableFetch<KIND>& tf, int tid) {
  if constexpr (FastTraits<KIND>::grid > 0) {
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const int i = tid + k * NT;
      if (i < FastTraits<KIND>::grid) t.grid[i] = u32x2{(uint32_t)tf.g[k], (uint32_t)(tf.g[k] >> 32)};
    }
  }
  if (tid < 16) {
    const u32x4 m = sign_masks((uint32_t)tid);
    t.sign4[tid] = u32x2{m[0], m[1]};
  }
  if constexpr (DirectKind<KIND>::pair_codes > 0) {
    if (tid < 256) t.kv2[tid] = tf.b;
  }
  if constexpr (FastTraits<KIND>::q2 > 0) {
    for (int i = tid; i < 256; i += NT)
      t.q2[i] = u32x2{pack_h2((float)(i & 3) - 1.0f, (float)((i >> 2) & 3) - 1.0f),
                      pack_h2((float)((i >> 4) & 3) - 1.0f, (float)(i >> 6) - 1.0f)};
  }
}

// The compiler no longer knows the fields' values: code that decodes them cannot move above this point.
template <int KIND>
__device__ __forceinline__ void opaque(RunPair<KIND>& f) {
  if constexpr (KIND == K_Q8_0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) asm volatile("" : "+v"(f.q[i]));
    asm volatile("" : "+v"(f.d[0]), "+v"(f.d[1]));
    return;
  } else if constexpr (KIND == K_Q4_K) {
    asm volatile("" : "+v"(f.qs[0]), "+v"(f.qs[1]), "+v"(f.sm), "+v"(f.dd));
    return;
  } else if constexpr (KIND == K_Q5_K) {
    asm volatile("" : "+v"(f.qs[0]), "+v"(f.qs[1]), "+v"(f.qh[0]), "+v"(f.qh[1]), "+v"(f.sm), "+v"(f.dd));
    return;
  } else if constexpr (KIND == K_Q6_K) {
    asm volatile("" : "+v"(f.ql[0]), "+v"(f.ql[1]), "+v"(f.qh[0]), "+v"(f.qh[1]), "+v"(f.sc[0]), "+v"(f.sc[1]),
                 "+v"(f.d));
    return;
  } else if constexpr (KIND == K_Q3_K) {
    asm volatile("" : "+v"(f.qs[0]), "+v"(f.qs[1]), "+v"(f.hm[0]), "+v"(f.hm[1]), "+v"(f.lo), "+v"(f.hi), "+v"(f.d));
    return;
  } else if constexpr (KIND == K_IQ4_XS) {
    asm volatile("" : "+v"(f.qs[0]), "+v"(f.qs[1]), "+v"(f.dh), "+v"(f.sl));
    return;
  } else if constexpr (KIND == K_IQ4_NL || KIND == K_Q4_0) {
    asm volatile("" : "+v"(f.qs[0]), "+v"(f.qs[1]), "+v"(f.d[0]), "+v"(f.d[1]));
    return;
  } else if constexpr (KIND == K_Q5_0) {
    asm volatile("" : "+v"(f.qs[0]), "+v"(f.qs[1]), "+v"(f.qh[0]), "+v"(f.qh[1]), "+v"(f.d[0]), "+v"(f.d[1]));
    return;
  } else {
#pragma unroll
  for (int i = 0; i < 4; ++i) asm volatile("" : "+v"(f.qs[i]));
  asm volatile("" : "+v"(f.d));
  }
  if constexpr (KIND == K_IQ3_S) {
    asm volatile("" : "+v"(f.qh), "+v"(f.sc), "+v"(f.sg[0]), "+v"(f.sg[1]));
  } else if constexpr (KIND == K_IQ3_XXS) {
    asm volatile("" : "+v"(f.aux[0]), "+v"(f.aux[1]));
  }
}

// The loads of these 32 registers are complete here (the compiler waits for them before this point).
__device__ __forceinline__ void arrived(uint32_t (&v)[32]) {
#pragma unroll
  for (int i = 0; i < 32; i += 8)
    asm volatile("" : "+v"(v[i]), "+v"(v[i + 1]), "+v"(v[i + 2]), "+v"(v[i + 3]), "+v"(v[i + 4]), "+v"(v[i + 5]),
                 "+v"(v[i + 6]), "+v"(v[i + 7]));
}

// These 32 registers hold nothing yet: an empty definition, so the compiler does not materialize a value for
// them on this path (it would otherwise zero all 32 where the other path loads them).
__device__ __forceinline__ void unset(uint32_t (&v)[32]) {
#pragma unroll
  for (int i = 0; i < 32; i += 8)
    asm volatile("" : "=v"(v[i]), "=v"(v[i + 1]), "=v"(v[i + 2]), "=v"(v[i + 3]), "=v"(v[i + 4]), "=v"(v[i + 5]),
                 "=v"(v[i + 6]), "=v"(v[i + 7]));
}

// the lowest pair left in the four masks, taken out; -1 when none is
__device__ __forceinline__ int take_lowest(uint64_t& m) {
  const int b = __ffsll((unsigned long long)m) - 1;
  m &= m - 1;
  return b;
}
__device__ __forceinline__ int take_member(uint64_t& m0, uint64_t& m1, uint64_t& m2, uint64_t& m3) {
  if (m0) return take_lowest(m0);
  if (m1) return 64 + take_lowest(m1);
  if (m2) return 128 + take_lowest(m2);
  if (m3) return 192 + take_lowest(m3);
  return -1;
}

// Per-lane byte offsets of a lane's run pair j within a row (the same for every row of a unit).
template <int KIND>
struct LaneOffsets {
  uint32_t d, qs, a, b, c;  // IQ3_S: d, qs, qh (a), signs (b), scale (c); IQ3_XXS: d, qs, aux (a); Q2_0: d, qs
};
template <int KIND>
__device__ __forceinline__ LaneOffsets<KIND> lane_offsets(int j) {
  LaneOffsets<KIND> o{};
  if constexpr (KIND == K_IQ3_S) {  // d @0, qs[64] @2, qh[8] @66, signs[32] @74, scales[4] @106
    const uint32_t b = (j >> 2) * 110, jj = j & 3;
    o.d = b;
    o.qs = b + 2 + 16 * jj;
    o.a = b + 66 + 2 * jj;
    o.b = b + 74 + 8 * jj;
    o.c = b + 106 + 2 * (jj >> 1);
  } else if constexpr (KIND == K_IQ3_XXS) {  // d @0, qs[64] @2, aux[8] (u32) @66
    const uint32_t b = (j >> 2) * 98, jj = j & 3;
    o.d = b;
    o.qs = b + 2 + 16 * jj;
    o.a = b + 66 + 8 * jj;
  } else if constexpr (KIND == K_Q8_0) {  // two blocks of 34: d @0, int8 q[32] @2
    o.d = j * 68;
    o.qs = j * 68 + 2;
  } else if constexpr (KIND == K_Q4_K) {  // d, dmin @0, scales[12] @4, qs[128] @16 (sub-blocks 2k, 2k + 1 @16 + 32k)
    const uint32_t b = (j >> 2) * 144, jj = j & 3;
    o.d = b;
    o.qs = b + 16 + 32 * jj;
    o.a = b + 4;
  } else if constexpr (KIND == K_Q5_K) {  // d, dmin @0, scales[12] @4, qh[32] @16, qs[128] @48
    const uint32_t b = (j >> 2) * 176, jj = j & 3;
    o.d = b;
    o.a = b + 4;
    o.b = b + 16;
    o.qs = b + 48 + 32 * jj;
  } else if constexpr (KIND == K_Q3_K) {  // hmask[32] @0, qs[64] @32, scales[12] @96, d @108
    const uint32_t b = (j >> 2) * 110, jj = j & 3;
    o.d = b + 108;
    o.qs = b + 32 + 32 * (jj >> 1);
    o.a = b;
    o.b = b + 96 + 4 * (jj & 1);
    o.c = b + 104;
  } else if constexpr (KIND == K_IQ4_NL || KIND == K_Q4_0) {  // two blocks of 18: d @0, qs[16] @2
    o.d = j * 36;
    o.qs = j * 36 + 2;
  } else if constexpr (KIND == K_Q5_0) {  // two blocks of 22: d @0, qh (u32) @2, qs[16] @6
    o.d = j * 44;
    o.a = j * 44 + 2;
    o.qs = j * 44 + 6;
  } else if constexpr (KIND == K_IQ4_XS) {  // d @0, scales_h @2, scales_l[4] @4, qs[128] @8 (run ib @8 + 16 ib)
    const uint32_t b = (j >> 2) * 136, jj = j & 3;
    o.d = b;
    o.a = b + 4;
    o.qs = b + 8 + 32 * jj;
  } else if constexpr (KIND == K_Q6_K) {  // ql[128] @0, qh[64] @128, int8 scales[16] @192, d @208
    const uint32_t b = (j >> 2) * 210, hh = (j >> 1) & 1, r0 = j & 1;
    o.d = b + 208;
    o.qs = b + 64 * hh + 32 * r0;
    o.a = b + 128 + 32 * hh;
    o.b = b + 192 + 8 * hh + 2 * r0;  // run r0's two scales; run r0 + 2's four bytes on
  } else {  // Q2_0: d @0, qs[16] @2
    o.d = j * 18;
    o.qs = j * 18 + 2;
  }
  return o;
}

// The row's run (32 weights) that half h of lane run pair j multiplies: 2j + h, except Q6_K, whose lane takes
// runs r0 and r0 + 2 of a half block (block j / 4, half (j / 2) % 2, r0 = j % 2).
template <int KIND>
__device__ __forceinline__ int run_of(int j, int h) {
  if constexpr (KIND == K_Q6_K) return 8 * (j >> 2) + 4 * ((j >> 1) & 1) + (j & 1) + 2 * h;
  return 2 * j + h;
}

// One token's activations in LDS: lane j's two runs (h = 0, 1) as 16-byte pieces 17 j + 4 h + i (i the piece
// within the run), so a lane's 128 bytes are contiguous and lanes sit 272 bytes apart: the 8 (16) lanes served
// in one cycle of a 16-byte LDS read fall on distinct banks at 128 (256) bytes a clock.
constexpr int kXPitch = 17;  // 16-byte slots a lane
template <int KIND>
__device__ __forceinline__ int x_slot(int c) {  // the slot of piece c of the row (c / 4: the run)
  const int r = c >> 2, i = c & 3;
  int j, h;  // the lane and half that multiply run r: the inverse of run_of
  if constexpr (KIND == K_Q6_K) {
    j = 4 * (r >> 3) + 2 * ((r >> 2) & 1) + (r & 1);
    h = (r >> 1) & 1;
  } else {
    j = r >> 1;
    h = r & 1;
  }
  return kXPitch * j + 4 * h + i;
}

// A load at base + off: base the same for the whole wave, off the lane's (global_load v, v_off, s_base).
template <typename T>
__device__ __forceinline__ T load_at(const uint8_t* base, uint32_t off) {
  typedef const __attribute__((address_space(1))) Unaligned<T> GlobalT;
  const __attribute__((address_space(1))) uint8_t* b = (const __attribute__((address_space(1))) uint8_t*)base;
  return ((GlobalT*)(b + off))->v;
}

template <int KIND>
__device__ __forceinline__ void load_fields(const uint8_t* row, uint32_t lo, const LaneOffsets<KIND>& o,
                                            RunPair<KIND>& f) {
  if constexpr (KIND == K_Q8_0) {
    f.d[0] = load_at<uint16_t>(row, lo + o.d);
    f.q[0] = load_at<u32x4>(row, lo + o.qs);
    f.q[1] = load_at<u32x4>(row, lo + o.qs + 16);
    f.d[1] = load_at<uint16_t>(row, lo + o.d + 34);
    f.q[2] = load_at<u32x4>(row, lo + o.qs + 34);
    f.q[3] = load_at<u32x4>(row, lo + o.qs + 50);
    return;
  } else if constexpr (KIND == K_Q4_K) {
    f.dd = load_at<uint32_t>(row, lo + o.d);
    f.sm = load_at<u32x4>(row, lo + o.a);
    f.qs[0] = load_at<u32x4>(row, lo + o.qs);
    f.qs[1] = load_at<u32x4>(row, lo + o.qs + 16);
    return;
  } else if constexpr (KIND == K_Q5_K) {
    f.dd = load_at<uint32_t>(row, lo + o.d);
    f.sm = load_at<u32x4>(row, lo + o.a);
    f.qs[0] = load_at<u32x4>(row, lo + o.qs);
    f.qs[1] = load_at<u32x4>(row, lo + o.qs + 16);
    f.qh[0] = load_at<u32x4>(row, lo + o.b);
    f.qh[1] = load_at<u32x4>(row, lo + o.b + 16);
    return;
  } else if constexpr (KIND == K_Q3_K) {
    f.d = load_at<uint16_t>(row, lo + o.d);
    f.lo = load_at<uint32_t>(row, lo + o.b);
    f.hi = load_at<uint32_t>(row, lo + o.c);
    f.qs[0] = load_at<u32x4>(row, lo + o.qs);
    f.qs[1] = load_at<u32x4>(row, lo + o.qs + 16);
    f.hm[0] = load_at<u32x4>(row, lo + o.a);
    f.hm[1] = load_at<u32x4>(row, lo + o.a + 16);
    return;
  } else if constexpr (KIND == K_IQ4_NL || KIND == K_Q4_0) {
    f.d[0] = load_at<uint16_t>(row, lo + o.d);
    f.qs[0] = load_at<u32x4>(row, lo + o.qs);
    f.d[1] = load_at<uint16_t>(row, lo + o.d + 18);
    f.qs[1] = load_at<u32x4>(row, lo + o.qs + 18);
    return;
  } else if constexpr (KIND == K_Q5_0) {
    f.d[0] = load_at<uint16_t>(row, lo + o.d);
    f.qh[0] = load_at<uint32_t>(row, lo + o.a);
    f.qs[0] = load_at<u32x4>(row, lo + o.qs);
    f.d[1] = load_at<uint16_t>(row, lo + o.d + 22);
    f.qh[1] = load_at<uint32_t>(row, lo + o.a + 22);
    f.qs[1] = load_at<u32x4>(row, lo + o.qs + 22);
    return;
  } else if constexpr (KIND == K_IQ4_XS) {
    f.dh = load_at<uint32_t>(row, lo + o.d);
    f.sl = load_at<uint32_t>(row, lo + o.a);
    f.qs[0] = load_at<u32x4>(row, lo + o.qs);
    f.qs[1] = load_at<u32x4>(row, lo + o.qs + 16);
    return;
  } else if constexpr (KIND == K_Q6_K) {
    f.d = load_at<uint16_t>(row, lo + o.d);
    f.sc[0] = load_at<uint16_t>(row, lo + o.b);
    f.sc[1] = load_at<uint16_t>(row, lo + o.b + 4);
    f.ql[0] = load_at<u32x4>(row, lo + o.qs);
    f.ql[1] = load_at<u32x4>(row, lo + o.qs + 16);
    f.qh[0] = load_at<u32x4>(row, lo + o.a);
    f.qh[1] = load_at<u32x4>(row, lo + o.a + 16);
    return;
  } else {
  f.d = load_at<uint16_t>(row, lo + o.d);
  f.qs = load_at<u32x4>(row, lo + o.qs);
  if constexpr (KIND == K_IQ3_S) {
    f.qh = load_at<uint16_t>(row, lo + o.a);
    f.sg = load_at<u32x2>(row, lo + o.b);
    f.sc = load_at<uint16_t>(row, lo + o.c);
  } else if constexpr (KIND == K_IQ3_XXS) {
    f.aux = load_at<u32x2>(row, lo + o.a);
  }
  }
}

// gfx950's row swaps between two registers: d = 16 exchanges the odd rows of 16 lanes of the first with the even
// rows of the second (v_permlane16_swap), d = 32 the upper 32 lanes of the first with the lower 32 of the second
// (v_permlane32_swap). Returns the two registers after the swap.
__device__ __forceinline__ void swap_rows(float a, float b, int d, float& a2, float& b2) {
  const auto r = d == 16 ? __builtin_amdgcn_permlane16_swap(__float_as_uint(a), __float_as_uint(b), false, false)
                         : __builtin_amdgcn_permlane32_swap(__float_as_uint(a), __float_as_uint(b), false, false);
  a2 = __uint_as_float(r[0]);
  b2 = __uint_as_float(r[1]);
}

// v from the lane whose index differs in bit d (d = 1, 2, 4, 8: DPP within rows of 16; 16, 32: a row swap). For
// d = 4 and 8 the partner is the mirror lane within 8 / 16 lanes, which also differs in bit d: a reduction or an
// exchange between the two halves needs only that.
template <bool SWAP = false>
__device__ __forceinline__ float lanes_apart(float v, int d) {
  const int b = __float_as_int(v);
  if (d == 1) return __int_as_float(__builtin_amdgcn_update_dpp(0, b, 0xB1, 0xF, 0xF, false));   // quad_perm 1032
  if (d == 2) return __int_as_float(__builtin_amdgcn_update_dpp(0, b, 0x4E, 0xF, 0xF, false));   // quad_perm 2301
  if (d == 4) return __int_as_float(__builtin_amdgcn_update_dpp(0, b, 0x141, 0xF, 0xF, false));  // row_half_mirror
  if (d == 8) return __int_as_float(__builtin_amdgcn_update_dpp(0, b, 0x140, 0xF, 0xF, false));  // row_mirror
  if (SWAP && (d == 16 || d == 32)) {  // after swapping v with itself: the first copy the lower rows', the second the upper's
    float lo, hi;
    swap_rows(v, v, d, lo, hi);
    const int lane = __builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));
    return (lane & d) ? lo : hi;
  }
  return __shfl_xor(v, d);
}

// a + a' where bit d of the lane is clear, b + b' where it is set (a', b': the registers of the lane whose index
// differs in bit d), for d = 16, 32: a row swap of a with b puts a's upper rows beside its lower ones and b's lower
// rows beside its upper ones, so the sum of the two registers after the swap is the answer in every lane.
__device__ __forceinline__ float sum_swapped(float a, float b, int d) {
  float a2, b2;
  swap_rows(a, b, d, a2, b2);
  return a2 + b2;
}

// N partial sums a lane (N row steps) over rows of L lanes -> the lanes of group ln / (L / N) hold the total of
// row step ln / (L / N). Exchange halves first (N - 1 moves), then reduce the one value left (log2(L / N)). The
// loops count up to a constant, so they unroll and every index is known (a run-time index would put the sums in
// scratch memory). SWAP: row swaps for d = 16, 32 (with two tokens a pass they push the kernel into spills).
template <int L, int N, bool SWAP>
__device__ __forceinline__ float reduce_steps(float (&v)[N], int ln) {
  constexpr int kHalvings = N >= 8 ? 3 : N >= 4 ? 2 : N >= 2 ? 1 : 0;
#pragma unroll
  for (int k = 0; k < kHalvings; ++k) {
    const int n = N >> k, d = (L / 2) >> k;
    const bool up = (ln & d) != 0;
#pragma unroll
    for (int i = 0; i < n / 2; ++i) {
      if (SWAP && d >= 16) {
        v[i] = sum_swapped(v[i], v[i + n / 2], d);
        continue;
      }
      const float send = up ? v[i] : v[i + n / 2];
      const float keep = up ? v[i + n / 2] : v[i];
      v[i] = keep + lanes_apart(send, d);
    }
  }
  float s = v[0];
#pragma unroll
  for (int d = L / N / 2; d >= 1; d /= 2) s = SWAP && d >= 16 ? sum_swapped(s, s, d) : s + lanes_apart(s, d);
  return s;
}

// Unit geometry: L lanes to a row (LT when known at compile time, else p.ct), p.rt rows of each matrix a unit,
// p.ntiles units to a matrix; the grid is (units of a matrix / kWaves, stacks taken as separate units (1 in
// paired mode), pairs), so a wave finds its unit without a division.
// Every load before the first wait has no branch around it: rows past the end and lanes past a row's run
// pairs load the last row / run pair again, and an expert id out of range loads expert 0's rows and writes NaN.
template <int KIND, bool GLU, bool PAIRED, int TT, int RU, int LT>
__global__ __launch_bounds__(kThreads, TT == 1 ? 4 : 3) void direct_decode_kernel(MatvecParams p) {
  __shared__ DirectTables<KIND> tab;
  __shared__ u32x4 xs[kXPitch * (kDMaxCols / 64)];  // one token's activations, when every wave multiplies it
  const int tid = threadIdx.x, lane = tid % 64;
  const int wave = __builtin_amdgcn_readfirstlane(tid / 64);
  const int L = LT > 0 ? LT : p.ct;
  const int side = 64 / L;  // rows side by side
  const int sub = lane / L, ln = lane % L;
  const int npr = p.runs / 2;
  const bool live = ln < npr;
  const int jp = min(ln, npr - 1);
  constexpr int kSteps = PAIRED ? RU / 2 : RU;  // row steps of each matrix

  const int tile = blockIdx.x * kWaves + wave;
  const bool in_range = tile < p.ntiles;
  const int pair = blockIdx.z, z0 = blockIdx.y;
  const int r0 = (in_range ? tile : 0) * p.rt;

  const uint8_t* m0;
  const uint8_t* m1 = nullptr;
  uint32_t expert = 0;
  bool bad = false;
  if (p.mode == MODE_EXPERT) {
    expert = p.idx[pair];
    bad = expert >= (uint64_t)p.experts;
    const int64_t off = (int64_t)(bad ? 0u : expert) * p.mat_bytes;
    m0 = p.blocks[PAIRED ? 0 : z0] + off;
    if (PAIRED) m1 = p.blocks[1] + off;
  } else if (p.mode == MODE_PTRS) {
    m0 = p.ptrs[pair];
  } else {
    m0 = p.blocks[z0];
  }

  // loads in the order they are waited for: the tables' constants and the pairs' ids, the activations, the rows
  TableFetch<KIND> tf;
  fetch_tables<KIND>(tf, tid);
  uint32_t e[4] = {0, 0, 0, 0};
  const int chunks = (p.pairs + 63) >> 6;  // 64 pair ids a ballot
  if (p.mode == MODE_EXPERT) {
#pragma unroll
    for (int c = 0; c < 4; ++c)
      if (c < chunks) e[c] = p.idx[min(64 * c + lane, p.pairs - 1)];
  }
  const bool one_x = p.mode == MODE_EXPERT && !GLU && p.share == p.pairs;  // every pair the same token
  // one token for the whole workgroup (one token's routed pairs, a window's first token): read once, coalesced,
  // into LDS; otherwise each lane reads its own 128 bytes
  const bool shared_x = !GLU && (one_x || p.mode == MODE_DENSE);
  uint32_t x[TT][32];
  const int q0 = p.mode == MODE_DENSE ? 0 : pair;
  u32x4 xv[2];
  if (shared_x) {
    const u32x4* src = reinterpret_cast<const u32x4*>(p.x);
#pragma unroll
    for (int k = 0; k < 2; ++k) xv[k] = src[min(tid + k * kThreads, p.cols / 8 - 1)];
    unset(x[0]);  // read from LDS after the barrier
  } else if constexpr (!GLU) {
    fast_load_x<false>(p, q0, run_of<KIND>(jp, 0), x[0]);
    fast_load_x<false>(p, q0, run_of<KIND>(jp, 1), x[0] + 16);
  }
  const LaneOffsets<KIND> lo = lane_offsets<KIND>(jp);
  RunPair<KIND> f[RU];
#pragma unroll
  for (int s = 0; s < RU; ++s) {
    const int rb = r0 + (PAIRED ? s / 2 : s) * side;  // the step's first row, the same for the whole wave
    const int rw = min(rb, p.rows - 1), rl = min(rb + sub, p.rows - 1);
    if constexpr (DirectKind<KIND>::linear && !PAIRED) {
      if (p.row_ids != nullptr) {  // listed rows (dense): an id past the matrix reads row 0 and writes NaN
        const uint32_t id = p.row_ids[rl];
        load_fields<KIND>(m0, (id < (uint32_t)p.src_rows ? id : 0u) * (uint32_t)p.row_bytes, lo, f[s]);
        continue;
      }
    }
    const uint8_t* row = (PAIRED && (s & 1) ? m1 : m0) + (int64_t)rw * p.row_bytes;
    load_fields<KIND>(row, (uint32_t)(rl - rw) * p.row_bytes, lo, f[s]);
    asm volatile("" ::: "memory");  // the steps' loads go out in step order: step 0 is decoded first
  }
  if constexpr (GLU) {  // silu(gate) * up waits for its loads: after the rows' have gone out
    fast_load_x<true>(p, q0, run_of<KIND>(jp, 0), x[0]);
    fast_load_x<true>(p, q0, run_of<KIND>(jp, 1), x[0] + 16);
  }
  // nothing above moves below this point, nothing below moves above it
  asm volatile("" : "+v"(e[0]), "+v"(e[1]), "+v"(e[2]), "+v"(e[3]), "+v"(tf.g[0]), "+v"(tf.g[1])::"memory");
  // the pairs naming this expert from this one on; a wave whose expert an earlier pair names has no work
  uint64_t mb0 = 0, mb1 = 0, mb2 = 0, mb3 = 0;
  bool valid = in_range;
  store_tables<KIND>(tab, tf, tid);
  if (shared_x) {
#pragma unroll
    for (int k = 0; k < 2; ++k)
      if (tid + k * kThreads < p.cols / 8) xs[x_slot<KIND>(tid + k * kThreads)] = xv[k];
  }
  if (p.mode == MODE_EXPERT && !bad) {
    bool earlier = false;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      if (c >= chunks) break;
      const uint64_t m = __ballot(64 * c + lane < p.pairs && e[c] == expert);
      const int lo_bits = pair - 64 * c;  // bits below are earlier pairs
      const uint64_t below = lo_bits <= 0 ? 0ull : (lo_bits >= 64 ? ~0ull : ((1ull << lo_bits) - 1));
      earlier |= (m & below) != 0;
      const uint64_t mine = m & ~below;
      if (c == 0) mb0 = mine;
      if (c == 1) mb1 = mine;
      if (c == 2) mb2 = mine;
      if (c == 3) mb3 = mine;
    }
    valid = valid && !earlier;
  }
  __syncthreads();
  if (!valid) return;
  if (shared_x) {
#pragma unroll
    for (int v = 0; v < 8; ++v) {
      const u32x4 c = xs[kXPitch * jp + v];
#pragma unroll
      for (int i = 0; i < 4; ++i) x[0][4 * v + i] = c[i];
    }
  }
  if (bad) {  // a pair naming no expert: NaN
    const f16 nan = (f16)__builtin_nanf("");
    for (int r = r0 + lane; r < min(r0 + p.rt, p.rows); r += 64) {
      const int64_t o = (int64_t)pair * p.rows + r;
      if (p.out[PAIRED ? 0 : z0] != nullptr) reinterpret_cast<f16*>(p.out[PAIRED ? 0 : z0])[o] = nan;
      if (PAIRED && p.out[1] != nullptr) reinterpret_cast<f16*>(p.out[1])[o] = nan;
      if (PAIRED) reinterpret_cast<f16*>(p.glu_out)[o] = nan;
    }
    return;
  }

  // the transposed reduction needs the row length at compile time and no more row steps than lanes to a row
  constexpr bool kFast = LT > 0 && RU <= LT;
  constexpr int G = kFast ? LT / RU : 1;  // lanes holding one row step's total after the reduction
  int done = 0;  // window: tokens done
  for (int pass = 0;; ++pass) {
    int q[TT];
    int nq = 0;
    if (p.mode == MODE_DENSE) {
      nq = max(0, min(TT, p.tokens - done));
#pragma unroll
      for (int t = 0; t < TT; ++t) q[t] = done + t;
      done += nq;
    } else if (p.mode == MODE_PTRS || one_x) {
      nq = pass == 0 ? 1 : 0;
#pragma unroll
      for (int t = 0; t < TT; ++t) q[t] = pair;
    } else {
#pragma unroll
      for (int t = 0; t < TT; ++t) {
        q[t] = take_member(mb0, mb1, mb2, mb3);
        nq += q[t] >= 0;
      }
    }
    if (nq == 0) break;
    if constexpr (GLU) {  // its activations are loaded after the rows: every row step is waited for at once
#pragma unroll
      for (int st = 0; st < RU; ++st) opaque(f[st]);
    }
    // A pass's other activations are waited for where they are loaded. A load still in flight past this branch
    // would be counted by every later wait, on the first pass too, and step 0's decode would then wait for all
    // the row loads; as it is, the wait before each row step's decode counts only the row loads after that
    // step's, and step 0 is decoded while the later steps' bytes are still arriving.
#pragma unroll
    for (int t = 0; t < TT; ++t) {
      if (t < nq && (pass > 0 || t > 0)) {
        fast_load_x<GLU>(p, q[t], run_of<KIND>(jp, 0), x[t]);
        fast_load_x<GLU>(p, q[t], run_of<KIND>(jp, 1), x[t] + 16);
        arrived(x[t]);
      }
    }
    float xsum[TT][2 * kXSums<KIND> + 1];  // the tokens' sums of x for biased runs, once a pass
#pragma unroll
    for (int t = 0; t < TT; ++t) {
      if constexpr (kBiasedRuns<KIND>) {
        if (t < nq) {
          x_sums<KIND>(x[t], xsum[t]);
          x_sums<KIND>(x[t] + 16, xsum[t] + kXSums<KIND>);
        }
      }
    }
    float acc[TT][RU];
    float sums[RU][TT];  // row sums of the run-time reduction
#pragma unroll
    for (int s = 0; s < RU; ++s) {
      const int r = r0 + (PAIRED ? s / 2 : s) * side + sub;
#pragma unroll
      for (int t = 0; t < TT; ++t) acc[t][s] = 0.0f;
      if constexpr (!GLU) opaque(f[s]);  // decoded anew each pass, each step once its own loads are in
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        uint32_t w[16];
        const RunScale rs = decode_run<KIND>(f[s], h, jp, w, tab);
#pragma unroll
        for (int t = 0; t < TT; ++t)
          if (t < nq) acc[t][s] += apply_run<KIND>(rs, w, x[t] + 16 * h, xsum[t] + kXSums<KIND> * h);
      }
#pragma unroll
      for (int t = 0; t < TT; ++t) {
        acc[t][s] = live && r < p.rows ? acc[t][s] : 0.0f;
        if constexpr (!kFast) {
          float v = acc[t][s];
          for (int o = L / 2; o >= 1; o /= 2) v += __shfl_xor(v, o, L);
          sums[s][t] = v;
        }
      }
    }
    if constexpr (kFast) {
      // one write sequence for every row of the unit: lane ln of group g = ln / G holds row step g's total
      const int g = ln / G;
      const bool writer = ln % (PAIRED ? 2 * G : G) == 0;
      const int k = PAIRED ? g / 2 : g;  // the row step of its matrix
      const int r = r0 + k * side + sub;
#pragma unroll
      for (int t = 0; t < TT; ++t) {
        if (t >= nq) continue;
        const float v = reduce_steps<LT, RU, TT == 1>(acc[t], ln);
        float h = 0.0f;
        f16 gq, uq;
        if constexpr (PAIRED) {  // gate in group 2k, up in group 2k + 1
          const float up = lanes_apart<TT == 1>(v, G);
          gq = from_f32<f16>(v);
          uq = from_f32<f16>(up);
          h = swiglu_rounded<f16>(gq, uq);
        }
        if (writer && r < p.rows) {
          uint64_t a0 = mb0, a1 = mb1, a2 = mb2, a3 = mb3;
          for (int qq = one_x ? take_member(a0, a1, a2, a3) : q[t]; qq >= 0;
               qq = one_x ? take_member(a0, a1, a2, a3) : -1) {
            const int64_t o = (int64_t)qq * p.rows + r;
            if constexpr (PAIRED) {
              if (p.out[0] != nullptr) reinterpret_cast<f16*>(p.out[0])[o] = gq;
              if (p.out[1] != nullptr) reinterpret_cast<f16*>(p.out[1])[o] = uq;
              reinterpret_cast<f16*>(p.glu_out)[o] = from_f32<f16>(h);
            } else {
              float vo = v;
              if constexpr (DirectKind<KIND>::linear)
                if (p.row_ids != nullptr && p.row_ids[r] >= (uint32_t)p.src_rows) vo = __builtin_nanf("");
              reinterpret_cast<f16*>(p.out[z0])[o] = from_f32<f16>(vo);
            }
          }
        }
      }
    } else {
      // lane 0 of each row writes: the pass's pairs, or (one token) every pair naming the expert
      if (ln == 0) {
#pragma unroll
        for (int kk = 0; kk < kSteps; ++kk) {
          const int r = r0 + kk * side + sub;
          if (r >= p.rows) continue;
#pragma unroll
          for (int t = 0; t < TT; ++t) {
            if (t >= nq) continue;
            uint64_t a0 = mb0, a1 = mb1, a2 = mb2, a3 = mb3;
            for (int qq = one_x ? take_member(a0, a1, a2, a3) : q[t]; qq >= 0;
                 qq = one_x ? take_member(a0, a1, a2, a3) : -1) {
              const int64_t o = (int64_t)qq * p.rows + r;
              if constexpr (PAIRED) {
                const f16 gg = from_f32<f16>(sums[2 * kk][t]), uu = from_f32<f16>(sums[2 * kk + 1][t]);
                if (p.out[0] != nullptr) reinterpret_cast<f16*>(p.out[0])[o] = gg;
                if (p.out[1] != nullptr) reinterpret_cast<f16*>(p.out[1])[o] = uu;
                reinterpret_cast<f16*>(p.glu_out)[o] = from_f32<f16>(swiglu_rounded<f16>(gg, uu));
              } else {
                float vo = sums[kk][t];
                if constexpr (DirectKind<KIND>::linear)
                  if (p.row_ids != nullptr && p.row_ids[r] >= (uint32_t)p.src_rows) vo = __builtin_nanf("");
                reinterpret_cast<f16*>(p.out[z0])[o] = from_f32<f16>(vo);
              }
            }
          }
        }
      }
    }
    if (p.mode != MODE_EXPERT && (p.mode == MODE_PTRS || (p.mode == MODE_DENSE && done >= p.tokens))) break;
    if (one_x) break;
    if (p.mode == MODE_EXPERT && (mb0 | mb1 | mb2 | mb3) == 0) break;
  }
}

// Row steps a unit takes: four, all loaded before the first is decoded (two gave half the fields in flight and
// were slower; eight hold three waves a SIMD).
constexpr int kRowSteps = 4;

template <int KIND, bool GLU, bool PAIRED, int TT, int RU, int LT>
int launch_direct_ru(MatvecParams& p, int grid_y, int grid_z, hipStream_t stream) {
  const int side = 64 / p.ct;
  p.tt = TT;
  p.nz = PAIRED ? 1 : grid_z;
  p.rt = (PAIRED ? RU / 2 : RU) * side;
  p.ntiles = (p.rows + p.rt - 1) / p.rt;
  if (grid_y > kDMaxGridY || p.nz > kDMaxGridY) return STRATA_ERR_SHAPE;
  p.items = p.ntiles;
  const dim3 grid((p.ntiles + kWaves - 1) / kWaves, p.nz, grid_y);
  hipLaunchKernelGGL((direct_decode_kernel<KIND, GLU, PAIRED, TT, RU, LT>), grid, dim3(kThreads), 0, stream, p);
  STRATA_CHECK_LAUNCH();
  return STRATA_OK;
}

// the row length at compile time for 4096 and 1536 inputs (64 and 32 lanes to a row), at run time otherwise
template <int KIND, bool GLU, bool PAIRED, int TT, int RU>
int launch_direct_lt(MatvecParams& p, int grid_y, int grid_z, hipStream_t s) {
  if (p.ct == 64) return launch_direct_ru<KIND, GLU, PAIRED, TT, RU, 64>(p, grid_y, grid_z, s);
  if (p.ct == 32) return launch_direct_ru<KIND, GLU, PAIRED, TT, RU, 32>(p, grid_y, grid_z, s);
  return launch_direct_ru<KIND, GLU, PAIRED, TT, RU, 0>(p, grid_y, grid_z, s);
}

template <int KIND, bool GLU, bool PAIRED, int TT>
int launch_direct_tt(MatvecParams& p, int grid_y, int grid_z, hipStream_t s) {
  // Q2_0 at two tokens a pass spills at four row steps (the compiler keeps more of its light decode in flight);
  // two steps give the same sums (each step's lanes meet by the same exchange)
  if constexpr (DirectKind<KIND>::linear) {  // their wider fields spill at four row steps
    return launch_direct_lt<KIND, GLU, PAIRED, TT, 2>(p, grid_y, grid_z, s);
  } else {
    if (kRowSteps == 2 || (KIND == K_Q2_0 && TT > 1))
      return launch_direct_lt<KIND, GLU, PAIRED, TT, 2>(p, grid_y, grid_z, s);
    return launch_direct_lt<KIND, GLU, PAIRED, TT, 4>(p, grid_y, grid_z, s);
  }
}

// Rows of 8 S run pairs for odd S (S = 3: 1536 inputs, the down projection of a 4096 x 1536 expert; S = 5: 2560)
// fill the power-of-two rows of direct_decode_kernel badly: 24 run pairs on 32 lanes leave a quarter of the lanes
// idle. Here 8 lanes take a row and lane m takes its run pairs m, m + 8, ... (S steps of eight consecutive run
// pairs, every lane busy), so a wave holds 8 rows, and a row's sum meets over 8 lanes by three DPP steps. The
// lane's activations differ from step to step: the pair's token sits in LDS (one copy for the workgroup, whose
// waves all multiply the same pair) and each step reads its 128 bytes. Routed pairs, a matrix a pair, or a window
// (its tokens one a pass, listed rows as in direct_decode_kernel), one token a pass.
template <int KIND, int S>
__global__ __launch_bounds__(kThreads, S <= 3 ? 4 : 3) void direct_odd_kernel(MatvecParams p) {
  constexpr int kPairs = 8 * S;     // run pairs of a row
  constexpr int kPieces = 8 * kPairs;  // 16-byte pieces of a token
  __shared__ DirectTables<KIND> tab;
  __shared__ u32x4 xs[kXPitch * kPairs];
  const int tid = threadIdx.x, lane = tid % 64;
  const int wave = __builtin_amdgcn_readfirstlane(tid / 64);
  const int m = lane & 7, sub = lane >> 3;  // run pairs m, m + 8, ... of row sub
  const int tile = blockIdx.x * kWaves + wave;
  const bool in_range = tile < p.ntiles;
  const int pair = blockIdx.z, z0 = blockIdx.y;
  const int r0 = (in_range ? tile : 0) * 8;
  const bool routed = p.mode == MODE_EXPERT, dense = p.mode == MODE_DENSE;
  const int rl = min(r0 + sub, p.rows - 1);  // the lane's output row
  uint32_t row = (uint32_t)rl;               // the matrix row it reads: a listed row's id (past the matrix: row 0)
  if (dense && p.row_ids != nullptr) {
    const uint32_t id = p.row_ids[rl];
    row = id < (uint32_t)p.src_rows ? id : 0u;
  }
  const uint32_t expert = routed ? p.idx[pair] : 0u;
  const bool bad = routed && expert >= (uint64_t)p.experts;
  const uint8_t* m0 = routed ? p.blocks[z0] + (int64_t)(bad ? 0u : expert) * p.mat_bytes
                             : dense ? p.blocks[z0] : p.ptrs[pair];

  // loads in the order they are waited for: the tables' constants and the pairs' ids, the token, the rows
  TableFetch<KIND> tf;
  fetch_tables<KIND>(tf, tid);
  uint32_t e[4] = {0, 0, 0, 0};
  const int chunks = (p.pairs + 63) >> 6;  // 64 pair ids a ballot
  if (routed) {
#pragma unroll
    for (int c = 0; c < 4; ++c)
      if (c < chunks) e[c] = p.idx[min(64 * c + lane, p.pairs - 1)];
  }
  const bool one_x = routed && p.share == p.pairs;  // every pair the same token: one pass writes them all
  u32x4 xv[(kPieces + kThreads - 1) / kThreads];
  const int x0 = dense ? 0 : pair / p.share;  // the first pass's token
  const u32x4* src = reinterpret_cast<const u32x4*>(reinterpret_cast<const f16*>(p.x) + (int64_t)x0 * p.cols);
#pragma unroll
  for (int k = 0; k * kThreads < kPieces; ++k) xv[k] = src[min(tid + k * kThreads, kPieces - 1)];
  RunPair<KIND> f[S];
#pragma unroll
  for (int s = 0; s < S; ++s) {
    load_fields<KIND>(m0, row * (uint32_t)p.row_bytes, lane_offsets<KIND>(8 * s + m), f[s]);
    asm volatile("" ::: "memory");  // the steps' loads go out in step order: step 0 is decoded first
  }
  asm volatile("" : "+v"(e[0]), "+v"(e[1]), "+v"(e[2]), "+v"(e[3]), "+v"(tf.g[0]), "+v"(tf.g[1])::"memory");
  store_tables<KIND>(tab, tf, tid);
#pragma unroll
  for (int k = 0; k * kThreads < kPieces; ++k)
    if (tid + k * kThreads < kPieces) xs[x_slot<KIND>(tid + k * kThreads)] = xv[k];
  // the pairs naming this expert from this one on (a matrix a pair: this pair); the same for every wave of the
  // workgroup (one pair)
  uint64_t mb[4] = {0, 0, 0, 0};
  bool earlier = false;
  if (!routed) {
#pragma unroll
    for (int c = 0; c < 4; ++c) mb[c] = pair / 64 == c ? 1ull << (pair % 64) : 0ull;
  } else if (!bad) {
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      if (c >= chunks) break;
      const uint64_t b = __ballot(64 * c + lane < p.pairs && e[c] == expert);
      const int lo_bits = pair - 64 * c;  // bits below are earlier pairs
      const uint64_t below = lo_bits <= 0 ? 0ull : (lo_bits >= 64 ? ~0ull : ((1ull << lo_bits) - 1));
      earlier |= (b & below) != 0;
      mb[c] = b & ~below;
    }
  }
  __syncthreads();
  if (earlier) return;  // an earlier pair's waves multiply these rows
  if (bad) {  // a pair naming no expert: NaN
    if (m == 0 && in_range && r0 + sub < p.rows)
      reinterpret_cast<f16*>(p.out[z0])[(int64_t)pair * p.rows + r0 + sub] = (f16)__builtin_nanf("");
    return;
  }
  for (int pass = 0;; ++pass) {
    // this pass's output row block: a window's token, or a pair naming the expert (the first: this one)
    const int q = dense ? (pass < p.tokens ? pass : -1) : take_member(mb[0], mb[1], mb[2], mb[3]);
    if (q < 0) break;
    if (pass > 0) {  // the next token into LDS, once every wave is done with the last one
      const int xq = dense ? q : q / p.share;
      const u32x4* sq = reinterpret_cast<const u32x4*>(reinterpret_cast<const f16*>(p.x) + (int64_t)xq * p.cols);
#pragma unroll
      for (int k = 0; k * kThreads < kPieces; ++k) xv[k] = sq[min(tid + k * kThreads, kPieces - 1)];
      __syncthreads();
#pragma unroll
      for (int k = 0; k * kThreads < kPieces; ++k)
        if (tid + k * kThreads < kPieces) xs[x_slot<KIND>(tid + k * kThreads)] = xv[k];
      __syncthreads();
    }
    float acc = 0.0f;
#pragma unroll
    for (int s = 0; s < S; ++s) {
      opaque(f[s]);  // decoded anew each pass, each step once its own loads are in
      const int j = 8 * s + m;
      uint32_t x[32];
#pragma unroll
      for (int v = 0; v < 8; ++v) {
        const u32x4 c = xs[kXPitch * j + v];
#pragma unroll
        for (int i = 0; i < 4; ++i) x[4 * v + i] = c[i];
      }
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        uint32_t w[16];
        const RunScale rs = decode_run<KIND>(f[s], h, j, w, tab);
        acc += apply_run<KIND>(rs, w, x + 16 * h);
      }
    }
    acc += lanes_apart(acc, 1);
    acc += lanes_apart(acc, 2);
    acc += lanes_apart(acc, 4);
    if (m == 0 && in_range && r0 + sub < p.rows) {  // this pass's pair, or (one token) every pair naming the expert
      if (dense && p.row_ids != nullptr && p.row_ids[rl] >= (uint32_t)p.src_rows) acc = __builtin_nanf("");  // past it
      const f16 v = from_f32<f16>(acc);
      f16* out = reinterpret_cast<f16*>(p.out[z0]) + r0 + sub;
      out[(int64_t)q * p.rows] = v;
      uint64_t a0 = mb[0], a1 = mb[1], a2 = mb[2], a3 = mb[3];
      if (one_x)
        for (int qq = take_member(a0, a1, a2, a3); qq >= 0; qq = take_member(a0, a1, a2, a3)) out[(int64_t)qq * p.rows] = v;
    }
    if (one_x) break;
  }
}

// Rows of 24 or 40 run pairs (1536, 2560 inputs), routed pairs or a matrix a pair, one token a pass:
// direct_odd_kernel.
template <int KIND>
int launch_direct_odd(MatvecParams& p, int grid_y, int grid_z, hipStream_t stream) {
  if constexpr (KIND == K_Q4_K || KIND == K_Q5_K || KIND == K_Q8_0) {
    return STRATA_ERR_SHAPE;
  } else {
    const int pairs = p.cols / 64;
    if (grid_y > kDMaxGridY || grid_z > kDMaxGridY ||
        (int64_t)std::max(p.rows, p.src_rows) * p.row_bytes >= ((int64_t)1 << 32))
      return STRATA_ERR_SHAPE;
    p.nz = grid_z;
    p.ntiles = (p.rows + 7) / 8;
    p.items = p.ntiles;
    const dim3 grid((p.ntiles + kWaves - 1) / kWaves, grid_z, grid_y);
    if (pairs == 24) {
      hipLaunchKernelGGL((direct_odd_kernel<KIND, 3>), grid, dim3(kThreads), 0, stream, p);
    } else if (pairs == 40) {
      hipLaunchKernelGGL((direct_odd_kernel<KIND, 5>), grid, dim3(kThreads), 0, stream, p);
    } else {
      return STRATA_ERR_SHAPE;
    }
    STRATA_CHECK_LAUNCH();
    return STRATA_OK;
  }
}

// Whether direct_odd_kernel takes the call: rows of 24 / 40 run pairs, one token a pass. The codebook types at
// both widths; Q3_K and Q6_K at 40 run pairs only (at 24, as fast as direct_decode_kernel's 32-lane rows); not
// Q8_0 (its five-step form holds three waves a SIMD and is slower) nor Q4_K (with its run sums of x it spills).
template <int KIND>
bool odd_takes(const MatvecParams& p) {
  if constexpr (KIND == K_Q4_K || KIND == K_Q5_K || KIND == K_Q8_0) return false;
  if (DirectKind<KIND>::linear && p.cols != 40 * 64) return false;
  // listed rows (dense): when the matrix's byte offsets fit 32 bits
  const bool ids_ok = p.row_ids == nullptr ||
                      (p.mode == MODE_DENSE && (int64_t)p.src_rows * p.row_bytes < ((int64_t)1 << 32));
  return p.cols % 64 == 0 && (p.cols / 64 == 24 || p.cols / 64 == 40) && ids_ok &&
         (p.mode == MODE_DENSE || p.pairs <= kDMaxPairs) && p.glu_out == nullptr;
}

// Rows of 64 to 4096 weights in run pairs (every IQ3_S / IQ3_XXS / Q2_0 row), up to 256 pairs.
inline bool direct_takes(const MatvecParams& p) {
  const int runs = p.cols / 32;
  return runs % 2 == 0 && runs >= 2 && runs / 2 <= 64 && (p.mode != MODE_EXPERT || p.pairs <= kDMaxPairs) &&
         (p.mode != MODE_PTRS || p.pairs <= kDMaxGridY);
}

template <int KIND, bool GLU, bool PAIRED>
int launch_direct(MatvecParams& p, bool one_token, int grid_y, int grid_z, hipStream_t s) {
  p.runs = p.cols / 32;
  int L = 1;
  while (L < p.runs / 2) L *= 2;
  p.ct = L;
  // the linear kinds take one token a pass (two spill), decoding their rows again for each token
  if (one_token || DirectKind<KIND>::linear) return launch_direct_tt<KIND, GLU, PAIRED, 1>(p, grid_y, grid_z, s);
  if constexpr (!DirectKind<KIND>::linear) return launch_direct_tt<KIND, GLU, PAIRED, 2>(p, grid_y, grid_z, s);
  return STRATA_ERR_SHAPE;
}

}  // namespace strata_mv

#include "routed_impl.h"
#include "stream_impl.h"

namespace strata_mv {

// The float16 fast paths where they apply (a type of FastTraits, float16 in and out, rows contiguous): the
// direct kernel, else the persistent wave kernel, else the staged fast kernel; other cases the generic kernels.
template <int KIND>
int launch_matvec_any(MatvecParams& p, int x_dtype, int out_dtype, bool glu, int grid_y, int grid_z, hipStream_t s) {
  // a shared expert in the routed launch: only the persistent routed forms take it
  if (p.shared[0] != nullptr) {
    if (!glu && x_dtype == DT_F16 && out_dtype == DT_F16 && grid_z == 2 && routed_glu_takes<KIND>(p))
      return launch_routed_glu<KIND>(p, s);
    if (!glu && x_dtype == DT_F16 && out_dtype == DT_F16 && grid_z == 1 && p.shared_x != nullptr &&
        routed_down_takes<KIND>(p))
      return launch_routed_down<KIND>(p, s);
    return STRATA_ERR_SHAPE;
  }
  // a float32 token against Q4_K rows of 4096 inputs: the persistent form, the token in two float16 parts
  if (!glu && x_dtype == DT_F32 && out_dtype == DT_F32 && routed_one32_takes<KIND>(p))
    return launch_routed_one<KIND, true>(p, s);
  if constexpr (DirectKind<KIND>::linear) {  // float16 in and out, rows of run pairs: the direct kernel
    // listed rows too (dense), when the matrix's byte offsets fit 32 bits: a listed row gets the bits of its
    // layer's full product
    const bool ids_ok = p.row_ids == nullptr ||
                        (p.mode == MODE_DENSE && (int64_t)p.src_rows * p.row_bytes < ((int64_t)1 << 32));
    if (x_dtype == DT_F16 && out_dtype == DT_F16 && ids_ok && direct_takes(p)) {
      const bool one = p.mode == MODE_PTRS || (p.mode == MODE_DENSE ? p.tokens == 1
                                                                     : (glu ? p.pairs <= 16
                                                                            : p.pairs <= p.share || p.pairs <= 8));
      if (!glu && stream_takes<KIND>(p, grid_y)) return launch_stream<KIND>(p, s);
      if (!glu && routed_one_takes<KIND>(p)) return launch_routed_one<KIND>(p, s);
      if (p.glu_out != nullptr) {
        if (!glu && grid_z == 2 && routed_glu_takes<KIND>(p)) return launch_routed_glu<KIND>(p, s);
        if (glu || grid_z != 2) return STRATA_ERR_SHAPE;
        return launch_direct<KIND, false, true>(p, one, grid_y, grid_z, s);
      }
      // one token a pass either way: rows of 24 / 40 run pairs on 8 lanes a row
      if (!glu && odd_takes<KIND>(p)) return launch_direct_odd<KIND>(p, grid_y, grid_z, s);
      return glu ? launch_direct<KIND, true, false>(p, one, grid_y, grid_z, s)
                 : launch_direct<KIND, false, false>(p, one, grid_y, grid_z, s);
    }
  }
  if constexpr (FastTraits<KIND>::supported) {
    if (x_dtype == DT_F16 && out_dtype == DT_F16 && p.row_ids == nullptr) {
      // one token a pass (four waves a SIMD) up to 64 routed pairs: most experts are named once, and the second
      // token a pass (three waves a SIMD) pays only where they are not (four tokens: 2458 against 2343 GB/s)
      const bool one = p.mode == MODE_PTRS || (p.mode == MODE_DENSE ? p.tokens == 1
                                                                     : (glu ? p.pairs <= 16
                                                                            : p.pairs <= p.share || p.pairs <= 64));
      if (p.glu_out != nullptr) {
        if (!glu && grid_z == 2 && routed_glu_takes<KIND>(p)) return launch_routed_glu<KIND>(p, s);
        if (!direct_takes(p) || glu || grid_z != 2) return STRATA_ERR_SHAPE;
        return launch_direct<KIND, false, true>(p, one, grid_y, grid_z, s);
      }
      if (!glu && grid_z == 1 && routed_down_takes<KIND>(p)) return launch_routed_down<KIND>(p, s);
      // the same for the 8-lane rows against two tokens a pass on 32-lane rows (four tokens: 2283 against 2047)
      if (!glu && one && odd_takes<KIND>(p)) return launch_direct_odd<KIND>(p, grid_y, grid_z, s);
      if (direct_takes(p)) {
        return glu ? launch_direct<KIND, true, false>(p, one, grid_y, grid_z, s)
                   : launch_direct<KIND, false, false>(p, one, grid_y, grid_z, s);
      }
      int rpl = 0;
      if ((p.mode == MODE_DENSE || p.pairs <= kPMaxPairs) && wave_lanes(p.cols / 32, &rpl) > 0) {
        return glu ? launch_wave_rpl<KIND, true>(p, one, grid_y, grid_z, s)
                   : launch_wave_rpl<KIND, false>(p, one, grid_y, grid_z, s);
      }
      if (glu) return one ? launch_fast<KIND, true, 1>(p, grid_y, grid_z, s) : launch_fast<KIND, true, 4>(p, grid_y, grid_z, s);
      return one ? launch_fast<KIND, false, 1>(p, grid_y, grid_z, s) : launch_fast<KIND, false, 4>(p, grid_y, grid_z, s);
    }
  }
  if (p.glu_out != nullptr) return STRATA_ERR_SHAPE;
  return launch_matvec_kind<KIND>(p, x_dtype, out_dtype, glu, grid_y, grid_z, s);
}

}  // namespace strata_mv
