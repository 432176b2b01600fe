// Shared definitions of the gfx950 library: block types, dtypes, small device helpers.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/strata_gfx950.h"

// GGUF type ids (strata_mlx/gguf.py:25-33); the C ABI takes a block type as one of these.
enum StrataKind : int {
  K_Q4_0 = 2, K_Q5_0 = 6, K_Q8_0 = 8, K_Q3_K = 11, K_Q4_K = 12, K_Q5_K = 13, K_Q6_K = 14,
  K_IQ2_XXS = 16, K_IQ2_XS = 17, K_IQ3_XXS = 18, K_IQ4_NL = 20, K_IQ3_S = 21, K_IQ2_S = 22,
  K_IQ4_XS = 23, K_IQ1_M = 29, K_Q2_0 = 42,
};

// weights and bytes per block of each type the kernels decode; 0 for a type they refuse
static inline int strata_kind_info(int kind, int* per_block, int* block_bytes) {
  int p = 0, b = 0;
  switch (kind) {
    case K_Q4_0: p = 32; b = 18; break;
    case K_Q5_0: p = 32; b = 22; break;
    case K_Q8_0: p = 32; b = 34; break;
    case K_Q3_K: p = 256; b = 110; break;
    case K_Q4_K: p = 256; b = 144; break;
    case K_Q6_K: p = 256; b = 210; break;
    case K_IQ3_XXS: p = 256; b = 98; break;
    case K_IQ4_NL: p = 32; b = 18; break;
    case K_IQ3_S: p = 256; b = 110; break;
    case K_IQ4_XS: p = 256; b = 136; break;
    case K_Q5_K: p = 256; b = 176; break;
    case K_Q2_0: p = 64; b = 18; break;
    default: return -1;
  }
  if (per_block) *per_block = p;
  if (block_bytes) *block_bytes = b;
  return 0;
}

// activations / outputs
enum StrataDtype : int { DT_F32 = STRATA_F32, DT_F16 = STRATA_F16, DT_BF16 = STRATA_BF16 };

typedef _Float16 f16;
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint16_t bf16_bits;

struct bf16_t {
  uint16_t bits;
};

__device__ __forceinline__ float to_f32(float v) { return v; }
__device__ __forceinline__ float to_f32(f16 v) { return (float)v; }
__device__ __forceinline__ float to_f32(bf16_t v) { return __uint_as_float((uint32_t)v.bits << 16); }

template <typename T>
__device__ __forceinline__ T from_f32(float v);
template <>
__device__ __forceinline__ float from_f32<float>(float v) { return v; }
// float32 -> float16, round to nearest even, fp16 subnormals included. Left to itself the compiler fuses
// the conversion into mixed-precision multiplies (v_fma_mix*, v_cvt_pk_f16_f32) that flush subnormal
// results to zero; the barrier keeps the float32 value as computed, and the subnormal range (|v| < 2^-14)
// is rounded here: v * 2^24 is exact and below 1024, and rint rounds it to nearest even.
template <>
__device__ __forceinline__ f16 from_f32<f16>(float v) {
  asm volatile("" : "+v"(v));
  const uint32_t u = __float_as_uint(v), a = u & 0x7fffffffu;
  if (a < 0x38800000u) {
    const uint32_t m = (uint32_t)__builtin_rintf(__uint_as_float(a) * 16777216.0f);
    return __builtin_bit_cast(f16, (uint16_t)(((u >> 16) & 0x8000u) | m));
  }
  return (f16)v;
}
template <>
__device__ __forceinline__ bf16_t from_f32<bf16_t>(float v) {
  uint32_t u = __float_as_uint(v);
  bf16_t r;
  if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu)) {
    r.bits = (uint16_t)((u >> 16) | 0x40);  // a NaN stays a quiet NaN
  } else {
    r.bits = (uint16_t)((u + 0x7fffu + ((u >> 16) & 1)) >> 16);  // round to nearest even
  }
  return r;
}

__device__ __forceinline__ float half_bits_to_f32(uint32_t h) {
  return (float)__builtin_bit_cast(f16, (uint16_t)h);
}

// The power of two that puts magnitude m (float bits) into [2^14, 2^15): floor(log2 m) - 14; 0 for m = 0, an
// infinity or a NaN. A row of activations scaled into float16 was divided by it.
__device__ __forceinline__ int row_exponent(uint32_t m) {
  m &= 0x7fffffffu;
  if (m == 0 || m >= 0x7f800000u) return 0;
  const int ex = (int)(m >> 23);
  const int lg = ex ? ex - 127 : (31 - __builtin_clz(m)) - 149;
  return lg - 14;
}

#define STRATA_CHECK_LAUNCH()                          \
  do {                                                 \
    hipError_t e_ = hipGetLastError();                 \
    if (e_ != hipSuccess) return STRATA_ERR_LAUNCH;    \
  } while (0)
