// The choice of the k largest logits of a row by one wave, ties to the lower index, and the softmax of the chosen
// (strata_mlx/fused.py:400-436, 490-491): shared by the top_k and router launches (fused.hip) and by the routed
// gate/up launch that makes its own choice of experts (routed_impl.h).
#pragma once

#include <math.h>

namespace strata_topk {

// (value, index) a over b: larger value, then lower index
__device__ __forceinline__ bool beats(float va, uint32_t ia, float vb, uint32_t ib) {
  return va > vb || (va == vb && ia < ib);
}

// v from a lane whose index differs in bit d, the other half of an aligned group of 2d lanes (d = 1, 2: quad
// permutes; 4, 8: the mirror lane within 8 / 16, by DPP; 16, 32: gfx950's row swap of v with itself, whose first
// copy then holds the lower rows' values and whose second the upper rows'): enough for a butterfly. No step goes
// through the LDS crossbar (a permute there took about a hundred cycles a step, eight rounds of two a top-8).
__device__ __forceinline__ uint32_t across(uint32_t v, int d) {
  if (d == 1) return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0xB1, 0xF, 0xF, false);   // quad_perm 1032
  if (d == 2) return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x4E, 0xF, 0xF, false);   // quad_perm 2301
  if (d == 4) return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x141, 0xF, 0xF, false);  // row_half_mirror
  if (d == 8) return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x140, 0xF, 0xF, false);  // row_mirror
  const auto r = d == 16 ? __builtin_amdgcn_permlane16_swap(v, v, false, false)
                         : __builtin_amdgcn_permlane32_swap(v, v, false, false);
  const uint32_t lane = __builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));
  return (lane & (uint32_t)d) ? r[0] : r[1];
}
__device__ __forceinline__ float across_f(float v, int d) { return __uint_as_float(across(__float_as_uint(v), d)); }

// One wave: the row's n <= 64 NV logits v (lane l holds logits l, l + 64, ...; -inf past n) -> the k largest into
// idx (k), their softmax into weights (k, or null); k <= 64.
template <int NV>
__device__ __forceinline__ void top_k_row(float (&v)[NV], int n, int k, int lane, uint32_t* __restrict__ idx,
                                          float* __restrict__ weights) {
  float chosen = 0.0f;  // lane q keeps the q-th chosen logit
  uint32_t taken = 0;
  for (int q = 0; q < k; ++q) {
    float best = -INFINITY;
    uint32_t at = 0xffffffffu;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const uint32_t j = (uint32_t)(i * 64 + lane);
      if ((int)j < n && beats(v[i], j, best, at)) {
        best = v[i];
        at = j;
      }
    }
#pragma unroll
    for (int o = 1; o <= 32; o *= 2) {
      const float ob = __uint_as_float(across(__float_as_uint(best), o));
      const uint32_t oa = across(at, o);
      if (beats(ob, oa, best, at)) {
        best = ob;
        at = oa;
      }
    }
    if (lane == q) {
      chosen = best;
      taken = at;
    }
    if (at != 0xffffffffu && (int)(at % 64) == lane) {
#pragma unroll
      for (int i = 0; i < NV; ++i)
        if (i == (int)(at / 64)) v[i] = -INFINITY;
    }
  }
  if (lane < k) idx[lane] = taken;
  if (weights != nullptr) {
    float m = lane < k ? chosen : -INFINITY;
#pragma unroll
    for (int o = 32; o >= 1; o /= 2) m = fmaxf(m, across_f(m, o));
    const float ex = lane < k ? expf(chosen - m) : 0.0f;
    float s = ex;
#pragma unroll
    for (int o = 32; o >= 1; o /= 2) s += across_f(s, o);
    if (lane < k) weights[lane] = ex / s;
  }
}

}  // namespace strata_topk
