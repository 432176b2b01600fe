// The decode matvec for float16 activations: weights decoded straight to float16 in registers.
//
// Every weight of these types is a per-run scale times a small integer (IQ3_S: +-grid value 1..15, IQ3_XXS:
// +-4..62, Q2_0: code - 1 in -1..2), exact in float16. A thread decodes its run's 32 integers as 16 packed
// float16 pairs: codebook entries come from an LDS table that already holds them as float16, and their signs
// are applied by XOR masks from a second LDS table indexed by the sign byte. v_dot2_f32_f16 multiplies each
// pair by the same pair of activations (exact products, float32 sums), and the run's scale multiplies the
// run's sum once. The activations stay packed in registers for the whole tile: 16 VGPRs a token.
//
// Layout of a workgroup, as the generic kernel's (matvec_impl.h): rt consecutive rows of one matrix, staged
// into LDS with 16-byte loads issued as soon as the expert is known; thread (c, l) takes run c of rows l,
// l + rs, ...; partial sums reduced in LDS. A pair whose expert an earlier pair names leaves its work to that
// pair's workgroup, which multiplies the rows by every pair naming the expert (up to TT per pass).
#pragma once
#include <stdlib.h>

#include "matvec_impl.h"

namespace strata_mv {

typedef _Float16 h2_t __attribute__((ext_vector_type(2)));

template <int KIND>
struct FastTraits {
  static constexpr bool supported = false;
  static constexpr int grid = 0, signs = 0, q2 = 0;
};
template <>
struct FastTraits<K_IQ3_S> {
  static constexpr bool supported = true;
  static constexpr int grid = 512, signs = 256, q2 = 0;
};
template <>
struct FastTraits<K_IQ3_XXS> {
  static constexpr bool supported = true;
  static constexpr int grid = 256, signs = 128, q2 = 0;
};
template <>
struct FastTraits<K_Q2_0> {
  static constexpr bool supported = true;
  static constexpr int grid = 0, signs = 0, q2 = 256;
};

template <int KIND>
struct FastTables {
  u32x2 grid[FastTraits<KIND>::grid > 0 ? FastTraits<KIND>::grid : 1];     // four float16 values an entry
  u32x4 signs[FastTraits<KIND>::signs > 0 ? FastTraits<KIND>::signs : 1];  // eight XOR masks (bit 15 of a half)
  u32x2 q2[FastTraits<KIND>::q2 > 0 ? FastTraits<KIND>::q2 : 1];           // a Q2_0 code byte: four (c - 1)
};

__device__ __forceinline__ uint32_t pack_h2(float a, float b) {
  return (uint32_t)__builtin_bit_cast(uint16_t, (f16)a) | ((uint32_t)__builtin_bit_cast(uint16_t, (f16)b) << 16);
}

// eight sign bits -> four dwords, bit 15 / 31 of each set when the weight is negative
__device__ __forceinline__ u32x4 sign_masks(uint32_t s) {
  u32x4 m;
#pragma unroll
  for (int i = 0; i < 4; ++i) m[i] = (((s >> (2 * i)) & 1u) << 15) | (((s >> (2 * i + 1)) & 1u) << 31);
  return m;
}

template <int KIND>
__device__ __forceinline__ void fast_load_tables(FastTables<KIND>& t, int tid, int nt) {
  if constexpr (FastTraits<KIND>::grid > 0) {
    for (int i = tid; i < FastTraits<KIND>::grid; i += nt) {
      const uint32_t g = KIND == K_IQ3_S ? kStrataIq3sGrid[i] : kStrataIq3xxsGrid[i];
      t.grid[i] = u32x2{pack_h2((float)(g & 255), (float)((g >> 8) & 255)),
                        pack_h2((float)((g >> 16) & 255), (float)(g >> 24))};
    }
  }
  if constexpr (FastTraits<KIND>::signs > 0) {
    for (int i = tid; i < FastTraits<KIND>::signs; i += nt)
      t.signs[i] = sign_masks(KIND == K_IQ3_XXS ? strata_ksign((uint32_t)i) : (uint32_t)i);
  }
  if constexpr (FastTraits<KIND>::q2 > 0) {
    for (int i = tid; i < 256; i += nt)
      t.q2[i] = u32x2{pack_h2((float)(i & 3) - 1.0f, (float)((i >> 2) & 3) - 1.0f),
                      pack_h2((float)((i >> 4) & 3) - 1.0f, (float)(i >> 6) - 1.0f)};
  }
}

__device__ __forceinline__ uint32_t lds_u32(const uint8_t* p) {
  uint32_t v;
  __builtin_memcpy(&v, p, 4);  // 2-byte aligned in LDS: gfx950 reads it in one ds_read_b32
  return v;
}

// Run n of a row as 16 packed float16 pairs of integers (natural order) and its scale.
template <int KIND>
__device__ __forceinline__ float fast_decode(const uint8_t* row, uint32_t n, uint32_t* w, const FastTables<KIND>& t) {
  if constexpr (KIND == K_IQ3_S) {  // strata_mlx/blocks.py:89-102
    const uint8_t* b = row + (n >> 3) * 110;
    const uint32_t ib = n & 7;
    const float scale =
        strata_half_at(b) * (float)(1 + 2 * (((uint32_t)b[106 + (ib >> 1)] >> (4 * (ib & 1))) & 15));
    const uint32_t qs0 = lds_u32(b + 2 + 8 * ib), qs1 = lds_u32(b + 6 + 8 * ib);
    const uint32_t qh = b[66 + ib];
    const uint32_t sg = lds_u32(b + 74 + 4 * ib);
#pragma unroll
    for (int l = 0; l < 8; ++l) {
      const uint32_t qs = l < 4 ? qs0 : qs1;
      const uint32_t idx = ((qs >> (8 * (l & 3))) & 255) | (((qh >> l) & 1) << 8);
      const u32x2 g = t.grid[idx];
      const u32x4 m = t.signs[(sg >> (8 * (l >> 1))) & 255];
      w[2 * l] = g[0] ^ m[(l & 1) * 2];
      w[2 * l + 1] = g[1] ^ m[(l & 1) * 2 + 1];
    }
    return scale;
  } else if constexpr (KIND == K_IQ3_XXS) {  // strata_mlx/blocks.py:103-116
    const uint8_t* b = row + (n >> 3) * 98;
    const uint32_t ib = n & 7;
    const uint32_t aux = lds_u32(b + 66 + 4 * ib);
    const float scale = strata_half_at(b) * (0.5f + (float)(aux >> 28)) * 0.5f;
    const uint32_t qs0 = lds_u32(b + 2 + 8 * ib), qs1 = lds_u32(b + 6 + 8 * ib);
#pragma unroll
    for (int l = 0; l < 8; ++l) {
      const uint32_t qs = l < 4 ? qs0 : qs1;
      const u32x2 g = t.grid[(qs >> (8 * (l & 3))) & 255];
      const u32x4 m = t.signs[(aux >> (7 * (l >> 1))) & 127];
      w[2 * l] = g[0] ^ m[(l & 1) * 2];
      w[2 * l + 1] = g[1] ^ m[(l & 1) * 2 + 1];
    }
    return scale;
  } else {  // Q2_0, strata_mlx/blocks.py:58-68
    const uint8_t* b = row + (n >> 1) * 18;
    const uint8_t* q = b + 2 + 8 * (n & 1);
    const uint32_t q0 = lds_u32(q), q1 = lds_u32(q + 4);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const u32x2 c = t.q2[((i < 4 ? q0 : q1) >> (8 * (i & 3))) & 255];
      w[2 * i] = c[0];
      w[2 * i + 1] = c[1];
    }
    return strata_half_at(b);
  }
}

__device__ __forceinline__ float dot16(const uint32_t* w, const uint32_t* x) {
  float s = 0.0f;
#pragma unroll
  for (int i = 0; i < 16; ++i)
    s = __builtin_amdgcn_fdot2(__builtin_bit_cast(h2_t, w[i]), __builtin_bit_cast(h2_t, x[i]), s, false);
  return s;
}

// 32 activations of run c as 16 packed float16 pairs; in GLU mode silu(g) * u rounded as mlx-lm rounds it
template <bool GLU>
__device__ __forceinline__ void fast_load_x(const MatvecParams& p, int q, int c, uint32_t* x) {
  if constexpr (GLU) {
    const u32x4* g4 = reinterpret_cast<const u32x4*>(reinterpret_cast<const f16*>(p.x) + (int64_t)q * p.cols + 32 * c);
    const u32x4* u4 = reinterpret_cast<const u32x4*>(reinterpret_cast<const f16*>(p.up) + (int64_t)q * p.cols + 32 * c);
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const u32x4 gv = g4[v], uv = u4[v];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const f16 g0 = __builtin_bit_cast(f16, (uint16_t)(gv[i] & 0xffff));
        const f16 g1 = __builtin_bit_cast(f16, (uint16_t)(gv[i] >> 16));
        const f16 u0 = __builtin_bit_cast(f16, (uint16_t)(uv[i] & 0xffff));
        const f16 u1 = __builtin_bit_cast(f16, (uint16_t)(uv[i] >> 16));
        const f16 h0 = from_f32<f16>(swiglu_rounded<f16>(g0, u0));
        const f16 h1 = from_f32<f16>(swiglu_rounded<f16>(g1, u1));
        x[4 * v + i] = (uint32_t)__builtin_bit_cast(uint16_t, h0) | ((uint32_t)__builtin_bit_cast(uint16_t, h1) << 16);
      }
    }
  } else {
    const int xrow = p.mode == MODE_DENSE ? q : q / p.share;
    const u32x4* s4 = reinterpret_cast<const u32x4*>(reinterpret_cast<const f16*>(p.x) + (int64_t)xrow * p.cols + 32 * c);
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const u32x4 xv = s4[v];
#pragma unroll
      for (int i = 0; i < 4; ++i) x[4 * v + i] = xv[i];
    }
  }
}

template <int KIND, bool GLU, int TT>
__global__ __launch_bounds__(kThreads, TT == 1 ? 6 : 3) void fast_kernel(MatvecParams p) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  FastTables<KIND>& tab = *reinterpret_cast<FastTables<KIND>*>(smem);
  uint32_t* queue = reinterpret_cast<uint32_t*>(smem + ((sizeof(FastTables<KIND>) + 15) & ~15));
  int* flag = reinterpret_cast<int*>(queue + kMaxQueue);
  uint8_t* stage = reinterpret_cast<uint8_t*>(queue + kMaxQueue + 4);
  float* red = reinterpret_cast<float*>(stage + p.stage_bytes);

  const int tid = threadIdx.x, nt = blockDim.x;
  const int z = blockIdx.z;
  const int r0 = blockIdx.x * p.rt;
  const int nr = min(p.rt, p.rows - r0);
  f16* out = reinterpret_cast<f16*>(p.out[z]);

  const uint8_t* mat;
  uint32_t expert = 0;
  const int first = p.mode == MODE_DENSE ? 0 : (int)blockIdx.y;
  if (p.mode == MODE_EXPERT) {
    expert = p.idx[first];
    if (expert >= (uint64_t)p.experts) {
      f16* o = out + (int64_t)first * p.rows;
      for (int r = r0 + tid; r < r0 + nr; r += nt) o[r] = (f16)__builtin_nanf("");
      return;
    }
    mat = p.blocks[z] + (int64_t)expert * p.mat_bytes;
  } else if (p.mode == MODE_PTRS) {
    mat = p.ptrs[first];
  } else {
    mat = p.blocks[z];
  }

  // staging loads first: their latency hides everything below
  const uint8_t* src = mat + (int64_t)r0 * p.row_bytes;
  const int len = nr * p.row_bytes;
  const uintptr_t lo = (uintptr_t)src, hi = lo + (uintptr_t)len;
  const uintptr_t a0 = (lo + 15) & ~(uintptr_t)15, a1 = hi & ~(uintptr_t)15;
  const int chunks = a1 > a0 ? (int)((a1 - a0) >> 4) : 0;
  constexpr int kLoads = 8;  // 16-byte loads a thread keeps in flight: 32 KB for the workgroup
  u32x4 v[kLoads];
#pragma unroll
  for (int i = 0; i < kLoads; ++i)
    if (tid + i * nt < chunks) v[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(a0) + tid + i * nt);

  fast_load_tables<KIND>(tab, tid, nt);
  // a pair whose expert an earlier pair names leaves the work to it
  int dup = 0;
  if (p.mode == MODE_EXPERT)
    for (int q = tid; q < first; q += nt) dup |= p.idx[q] == expert;
  if (__syncthreads_or(dup)) return;

  uint8_t* base = stage + (lo & 15) - lo;  // LDS address of global byte g is base + g
#pragma unroll
  for (int i = 0; i < kLoads; ++i)
    if (tid + i * nt < chunks) reinterpret_cast<u32x4*>(base + a0)[tid + i * nt] = v[i];
  if (a0 > a1) {
    for (uintptr_t g = lo + tid; g < hi; g += nt) base[g] = *(const uint8_t*)g;
  } else {
    for (uintptr_t g = lo + tid; g < a0; g += nt) base[g] = *(const uint8_t*)g;
    for (uintptr_t g = a1 + tid; g < hi; g += nt) base[g] = *(const uint8_t*)g;
  }
  const uint8_t* rows0 = stage + (lo & 15);

  const int c = tid % p.ct, lane_row = tid / p.ct;
  const bool active = lane_row < p.rs;
  int scan = first, done = 0;
  for (;;) {
    // the next pairs of this expert (or tokens of the window), up to TT, in order
    int nq = 0;
    {
      __syncthreads();
      if (tid < 64) {
        int n = 0;
        if (p.mode == MODE_DENSE) {
          n = max(0, min(TT, p.tokens - done));
          if (tid < n) queue[tid] = done + tid;
        } else if (p.mode == MODE_PTRS) {
          n = done == 0 ? 1 : 0;
          if (tid == 0) queue[0] = first;
        } else {
          while (scan < p.pairs && n < TT) {  // 64 pairs at a time, wave ballots keep the order
            const int q = scan + tid;
            const bool hit = q < p.pairs && p.idx[q] == expert;
            const uint64_t m = __ballot(hit);
            const int before = __popcll(m & ((1ull << tid) - 1));
            if (hit && n + before < TT) queue[n + before] = q;
            const int take = min(__popcll(m), TT - n);
            if (take < __popcll(m)) {  // stop after the TT-th hit: resume there next pass
              uint64_t mm = m;
              for (int k = 0; k < take; ++k) mm &= mm - 1;
              scan += __ffsll((unsigned long long)mm) - 1;
              n += take;
              break;
            }
            n += take;
            scan += 64;
          }
        }
        if (tid == 0) *flag = n;
      }
      __syncthreads();
      nq = *flag;
      if (nq == 0) break;
    }
    done += nq;

    const int stride = p.ct + 1;
    if (active) {
      uint32_t x[TT][16];
#pragma unroll
      for (int t = 0; t < TT; ++t)
        if (t < nq) fast_load_x<GLU>(p, (int)queue[t], c, x[t]);
#pragma unroll 1
      for (int r = lane_row; r < nr; r += p.rs) {  // partial sums straight to LDS: no accumulator array
        uint32_t w[16];
        const float scale = fast_decode<KIND>(rows0 + r * p.row_bytes, (uint32_t)c, w, tab);
#pragma unroll
        for (int t = 0; t < TT; ++t)
          if (t < nq) red[(t * p.rt + r) * stride + c] = scale * dot16(w, x[t]);
      }
    }
    __syncthreads();
    const int outputs = nq * nr;
    for (int o = tid / 8; o < (outputs + (nt / 8) - 1) / (nt / 8) * (nt / 8); o += nt / 8) {
      float s = 0.0f;
      int t = 0, r = 0;
      if (o < outputs) {
        t = o / nr;
        r = o % nr;
        const float* vv = red + (t * p.rt + r) * stride;
        for (int cc = tid % 8; cc < p.ct; cc += 8) s += vv[cc];
      }
      s += __shfl_xor(s, 4, 8);
      s += __shfl_xor(s, 2, 8);
      s += __shfl_xor(s, 1, 8);
      if (o < outputs && tid % 8 == 0) out[(int64_t)queue[t] * p.rows + r0 + r] = from_f32<f16>(s);
    }
    if (p.mode == MODE_PTRS) break;
  }
}


// Rows a thread takes per tile, at most (fewer where the staged rows or the sums would not fit LDS).
constexpr int kFastRowsPerLane = kRowsPerLane;

// LDS: tables, queue, at most 32 KB of staged rows (what kLoads loads a thread cover), partial sums; 64 KB in all
template <int KIND, int TT>
inline int fast_geometry(MatvecParams& p, size_t* smem) {
  p.runs = p.cols / 32;
  if (p.runs < 1 || p.runs > kThreads) return STRATA_ERR_SHAPE;
  p.ct = p.runs;
  p.rs = kThreads / p.ct;
  const size_t fixed = ((sizeof(FastTables<KIND>) + 15) & ~(size_t)15) + (kMaxQueue + 4) * sizeof(uint32_t);
  for (int rpl = kFastRowsPerLane; rpl >= 1; rpl /= 2) {
    p.rt = p.rs * rpl;
    p.stage_bytes = ((p.rt * p.row_bytes + 32) + 15) & ~15;
    const size_t red = (size_t)TT * p.rt * (p.ct + 1) * sizeof(float);
    *smem = fixed + p.stage_bytes + red;
    if (p.rt * p.row_bytes + 16 <= 8 * kThreads * 16 && *smem <= 65536) return STRATA_OK;
  }
  return STRATA_ERR_SHAPE;
}

template <int KIND, bool GLU, int TT>
int launch_fast(MatvecParams& p, int grid_y, int grid_z, hipStream_t stream) {
  size_t smem = 0;
  int rc = fast_geometry<KIND, TT>(p, &smem);
  if (rc) return rc;
  p.tt = TT;
  dim3 grid((p.rows + p.rt - 1) / p.rt, grid_y, grid_z);
  hipLaunchKernelGGL((fast_kernel<KIND, GLU, TT>), grid, dim3(kThreads), smem, stream, p);
  STRATA_CHECK_LAUNCH();
  return STRATA_OK;
}

// The float16 fast path where it applies (a type of FastTraits, float16 in and out, rows contiguous), else the
// generic kernels. One token's pairs (or a window of one token) hold one token a pass, others four.
}  // namespace strata_mv
