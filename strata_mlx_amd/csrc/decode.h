// Device decoders: the n-th run of 32 weights of a row of blocks, as exact float32 values.
//
// One function per block type, each a restatement of that type's decode (strata_mlx/blocks.py:57-194
// for the expert types, strata_mlx/gguf.py:150-276 for the dense ones). Every value is an fp16 scale
// times small integers, exact in float32, so the order of the products does not matter; Q4_K is
// code * (d * sc) + -(dmin * mn), one rounding, with or without a fused multiply-add.
//
// `row` may point into LDS or global memory. Codebooks come from an LDS copy (StrataTables) that a
// kernel fills at its start (strata_load_tables).
#pragma once
#include "common.h"
#include "tables.h"

struct StrataTables {
  uint32_t grid[512];   // IQ3_S (512 entries) or IQ3_XXS (256): four weights a uint32, low byte first
  int32_t kvalues[16];  // IQ4_NL / IQ4_XS codebook
};

template <int KIND>
struct KindTraits;
#define STRATA_TRAITS(K, P, B, G, KV)                                                   \
  template <>                                                                           \
  struct KindTraits<K> {                                                                \
    static constexpr int per_block = P, block_bytes = B, grid_entries = G, kvalues = KV; \
  };
STRATA_TRAITS(K_Q2_0, 64, 18, 0, 0)
STRATA_TRAITS(K_IQ4_NL, 32, 18, 0, 1)
STRATA_TRAITS(K_IQ4_XS, 256, 136, 0, 1)
STRATA_TRAITS(K_IQ3_S, 256, 110, 512, 0)
STRATA_TRAITS(K_IQ3_XXS, 256, 98, 256, 0)
STRATA_TRAITS(K_Q3_K, 256, 110, 0, 0)
STRATA_TRAITS(K_Q4_K, 256, 144, 0, 0)
STRATA_TRAITS(K_Q5_K, 256, 176, 0, 0)
STRATA_TRAITS(K_Q6_K, 256, 210, 0, 0)
STRATA_TRAITS(K_Q8_0, 32, 34, 0, 0)
STRATA_TRAITS(K_Q4_0, 32, 18, 0, 0)
STRATA_TRAITS(K_Q5_0, 32, 22, 0, 0)
#undef STRATA_TRAITS

// Fill the kind's codebooks into LDS; every thread of the block calls it, then a barrier is due.
template <int KIND>
__device__ __forceinline__ void strata_load_tables(StrataTables& t) {
  constexpr int G = KindTraits<KIND>::grid_entries;
  for (int i = threadIdx.x + threadIdx.y * blockDim.x; i < G; i += blockDim.x * blockDim.y) {
    t.grid[i] = KIND == K_IQ3_S ? kStrataIq3sGrid[i] : kStrataIq3xxsGrid[i];
  }
  if (KindTraits<KIND>::kvalues) {
    int i = threadIdx.x + threadIdx.y * blockDim.x;
    if (i < 16) t.kvalues[i] = kStrataKvaluesIq4nl[i];
  }
}

__device__ __forceinline__ float strata_half_at(const uint8_t* b) {
  return half_bits_to_f32((uint32_t)b[0] | ((uint32_t)b[1] << 8));
}
__device__ __forceinline__ uint32_t strata_u16_at(const uint8_t* b) {
  return (uint32_t)b[0] | ((uint32_t)b[1] << 8);
}
__device__ __forceinline__ uint32_t strata_u32_at(const uint8_t* b) {
  return strata_u16_at(b) | (strata_u16_at(b + 2) << 16);
}
// ggml's ksigns_iq2xs[i]: seven stored sign bits and their parity as the eighth
__device__ __forceinline__ uint32_t strata_ksign(uint32_t i) { return i | ((uint32_t)(__popc(i) & 1) << 7); }

// strata_mlx/blocks.py:49-53
__device__ __forceinline__ float strata_q3k_scale(const uint8_t* s, uint32_t k) {
  uint32_t p = k % 4, word = k / 4;
  uint32_t low = word < 2 ? (s[4 * word + p] & 15u) : ((uint32_t)s[4 * (word - 2) + p] >> 4);
  return (float)((int)(low | ((((uint32_t)s[8 + p] >> (2 * word)) & 3u) << 4)) - 32);
}

template <int KIND>
__device__ __forceinline__ void strata_unpack32(const uint8_t* row, uint32_t n, float* w, const StrataTables& t) {
  if constexpr (KIND == K_Q2_0) {  // blocks.py:58-68
    const uint8_t* b = row + (n / 2) * 18;
    const uint8_t* q = b + 2 + 8 * (n % 2);
    float d = strata_half_at(b);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      uint32_t c = q[i];
#pragma unroll
      for (int j = 0; j < 4; ++j) w[4 * i + j] = d * ((float)((c >> (2 * j)) & 3) - 1.0f);
    }
  } else if constexpr (KIND == K_IQ4_NL) {  // blocks.py:69-77
    const uint8_t* b = row + n * 18;
    float d = strata_half_at(b);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      uint32_t q = b[2 + i];
      w[i] = d * (float)t.kvalues[q & 15];
      w[16 + i] = d * (float)t.kvalues[q >> 4];
    }
  } else if constexpr (KIND == K_IQ4_XS) {  // blocks.py:78-88
    const uint8_t* b = row + (n / 8) * 136;
    uint32_t ib = n % 8;
    uint32_t ls = (((uint32_t)b[4 + ib / 2] >> (4 * (ib % 2))) & 15) | (((strata_u16_at(b + 2) >> (2 * ib)) & 3) << 4);
    float d = strata_half_at(b) * ((float)ls - 32.0f);
    const uint8_t* q = b + 8 + 16 * ib;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      uint32_t v = q[i];
      w[i] = d * (float)t.kvalues[v & 15];
      w[16 + i] = d * (float)t.kvalues[v >> 4];
    }
  } else if constexpr (KIND == K_IQ3_S) {  // blocks.py:89-102
    const uint8_t* b = row + (n / 8) * 110;
    uint32_t ib = n % 8;
    float d = strata_half_at(b) * (float)(1 + 2 * (((uint32_t)b[106 + ib / 2] >> (4 * (ib % 2))) & 15));
    uint32_t high = b[66 + ib];
#pragma unroll
    for (int l = 0; l < 8; ++l) {
      uint32_t g = t.grid[(uint32_t)b[2 + 8 * ib + l] | (((high >> l) & 1) << 8)];
      uint32_t sign = (uint32_t)b[74 + 4 * ib + l / 2] >> (4 * (l % 2));
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        float v = d * (float)((g >> (8 * j)) & 255);
        w[4 * l + j] = ((sign >> j) & 1) ? -v : v;
      }
    }
  } else if constexpr (KIND == K_IQ3_XXS) {  // blocks.py:103-116
    const uint8_t* b = row + (n / 8) * 98;
    uint32_t ib = n % 8;
    uint32_t aux = strata_u32_at(b + 66 + 4 * ib);
    float d = strata_half_at(b) * (0.5f + (float)(aux >> 28)) * 0.5f;
#pragma unroll
    for (int l = 0; l < 8; ++l) {
      uint32_t g = t.grid[b[2 + 8 * ib + l]];
      uint32_t sign = strata_ksign((aux >> (7 * (l / 2))) & 127) >> (4 * (l % 2));
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        float v = d * (float)((g >> (8 * j)) & 255);
        w[4 * l + j] = ((sign >> j) & 1) ? -v : v;
      }
    }
  } else if constexpr (KIND == K_Q3_K) {  // blocks.py:164-175
    const uint8_t* b = row + (n / 8) * 110;
    uint32_t r = n % 8;
    const uint8_t* q = b + 32 + 32 * (r / 4);
    uint32_t shift = 2 * (r % 4);
    float d = strata_half_at(b + 108);
    float s0 = d * strata_q3k_scale(b + 96, 2 * r), s1 = d * strata_q3k_scale(b + 96, 2 * r + 1);
#pragma unroll
    for (int i = 0; i < 32; ++i) {
      int v = (int)(((uint32_t)q[i] >> shift) & 3) - ((((uint32_t)b[i] >> r) & 1) ? 0 : 4);
      w[i] = (i < 16 ? s0 : s1) * (float)v;
    }
  } else if constexpr (KIND == K_Q4_K) {  // gguf.py:174-179, 207-213; a run is a sub-block
    const uint8_t* b = row + (n / 8) * 144;
    uint32_t s = n % 8;
    const uint8_t* p = b + 4;
    uint32_t sc = s < 4 ? (p[s] & 63u) : ((p[s + 4] & 15u) | (((uint32_t)p[s - 4] >> 6) << 4));
    uint32_t mn = s < 4 ? (p[s + 4] & 63u) : (((uint32_t)p[s + 4] >> 4) | (((uint32_t)p[s] >> 6) << 4));
    float scale = strata_half_at(b) * (float)sc, bias = -(strata_half_at(b + 2) * (float)mn);
    const uint8_t* q = b + 16 + 32 * (s / 2);
#pragma unroll
    for (int i = 0; i < 32; ++i) {
      uint32_t code = (s % 2) ? ((uint32_t)q[i] >> 4) : (q[i] & 15u);
      w[i] = __builtin_fmaf((float)code, scale, bias);  // code * scale is exact: one rounding either way
    }
  } else if constexpr (KIND == K_Q5_K) {  // gguf.py:207-218: Q4_K's form, a fifth code bit from qh
    const uint8_t* b = row + (n / 8) * 176;
    uint32_t s = n % 8;
    const uint8_t* p = b + 4;
    uint32_t sc = s < 4 ? (p[s] & 63u) : ((p[s + 4] & 15u) | (((uint32_t)p[s - 4] >> 6) << 4));
    uint32_t mn = s < 4 ? (p[s + 4] & 63u) : (((uint32_t)p[s + 4] >> 4) | (((uint32_t)p[s] >> 6) << 4));
    float scale = strata_half_at(b) * (float)sc, bias = -(strata_half_at(b + 2) * (float)mn);
    const uint8_t* qh = b + 16;
    const uint8_t* q = b + 48 + 32 * (s / 2);
#pragma unroll
    for (int i = 0; i < 32; ++i) {
      uint32_t code = ((s % 2) ? ((uint32_t)q[i] >> 4) : (q[i] & 15u)) | ((((uint32_t)qh[i] >> s) & 1u) << 4);
      w[i] = __builtin_fmaf((float)code, scale, bias);  // code * scale is exact: one rounding either way
    }
  } else if constexpr (KIND == K_Q6_K) {  // gguf.py:150-165
    const uint8_t* b = row + (n / 8) * 210;
    uint32_t r8 = n % 8, h = r8 / 4, r = r8 % 4;
    const uint8_t* ql = b + 64 * h + (r & 1) * 32;
    const uint8_t* qh = b + 128 + 32 * h;
    float d = strata_half_at(b + 208);
    float s0 = d * (float)(int8_t)b[192 + 8 * h + 2 * r], s1 = d * (float)(int8_t)b[192 + 8 * h + 2 * r + 1];
#pragma unroll
    for (int i = 0; i < 32; ++i) {
      uint32_t lo = (r & 2) ? ((uint32_t)ql[i] >> 4) : (ql[i] & 15u);
      uint32_t hi = ((uint32_t)qh[i] >> (2 * r)) & 3;
      w[i] = (float)((int)(lo | (hi << 4)) - 32) * (i < 16 ? s0 : s1);
    }
  } else if constexpr (KIND == K_Q8_0) {  // gguf.py:203-206
    const uint8_t* b = row + n * 34;
    float d = strata_half_at(b);
#pragma unroll
    for (int i = 0; i < 32; ++i) w[i] = d * (float)(int8_t)b[2 + i];
  } else if constexpr (KIND == K_Q4_0) {  // gguf.py:195-197
    const uint8_t* b = row + n * 18;
    float d = strata_half_at(b);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      w[i] = d * (float)((int)(b[2 + i] & 15) - 8);
      w[16 + i] = d * (float)((int)(b[2 + i] >> 4) - 8);
    }
  } else if constexpr (KIND == K_Q5_0) {  // gguf.py:198-202
    const uint8_t* b = row + n * 22;
    float d = strata_half_at(b);
    uint32_t qh = strata_u32_at(b + 2);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      uint32_t lo = (b[6 + i] & 15u) | (((qh >> i) & 1) << 4);
      uint32_t hi = ((uint32_t)b[6 + i] >> 4) | (((qh >> (16 + i)) & 1) << 4);
      w[i] = d * (float)((int)lo - 16);
      w[16 + i] = d * (float)((int)hi - 16);
    }
  }
}

// Dispatch a runtime block type to a template instantiation: F(KindTag<K>{}) for the matching K.
template <int K>
struct KindTag {
  static constexpr int value = K;
};

template <typename F>
static inline int strata_dispatch_kind(int kind, F&& f) {
  switch (kind) {
    case K_Q2_0: return f(KindTag<K_Q2_0>{});
    case K_IQ4_NL: return f(KindTag<K_IQ4_NL>{});
    case K_IQ4_XS: return f(KindTag<K_IQ4_XS>{});
    case K_Q5_K: return f(KindTag<K_Q5_K>{});
    case K_IQ3_S: return f(KindTag<K_IQ3_S>{});
    case K_IQ3_XXS: return f(KindTag<K_IQ3_XXS>{});
    case K_Q3_K: return f(KindTag<K_Q3_K>{});
    case K_Q4_K: return f(KindTag<K_Q4_K>{});
    case K_Q6_K: return f(KindTag<K_Q6_K>{});
    case K_Q8_0: return f(KindTag<K_Q8_0>{});
    case K_Q4_0: return f(KindTag<K_Q4_0>{});
    case K_Q5_0: return f(KindTag<K_Q5_0>{});
    default: return STRATA_ERR_KIND;
  }
}

template <typename F>
static inline int strata_dispatch_dtype(int dtype, F&& f) {
  switch (dtype) {
    case DT_F32: return f((float*)nullptr);
    case DT_F16: return f((f16*)nullptr);
    case DT_BF16: return f((bf16_t*)nullptr);
    default: return STRATA_ERR_DTYPE;
  }
}
