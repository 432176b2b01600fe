// The persistent decode matvec for float16 activations (IQ3_S, IQ3_XXS, Q2_0): every wave works alone.
//
// A launch is a list of work items, each a few consecutive rows of one matrix: (pair, stack, rows) for the routed
// form, (stack, rows) for one layer's window, (pair, rows) for the per-pair pointer form. A few workgroups per CU
// build the LDS codebooks and the pairs' expert ids once (the only block barriers); after that every wave takes
// items round robin on its own, with its own slice of LDS:
//   - the next item's bytes are loaded into registers (16-byte loads, coalesced over the item) while the current
//     item is decoded, so a wave always has an item's bytes in flight;
//   - a row's runs of 32 weights are spread over L lanes (64, 32 or 16; up to four runs a lane), so 64 / L rows
//     are decoded side by side; each lane holds the activations of its runs in registers;
//   - a row's partial sums meet across its L lanes by shuffles, and one lane writes the row's output.
// A pair whose expert an earlier pair names has no items: the first pair's items multiply the rows by every pair
// naming the expert, TT a pass. Activations that do not change from item to item (one token's gate/up, a window
// of at most TT tokens) are loaded once.
//
// IQ3_S indices: each group of four weights has an eight-bit index in qs and a ninth bit in qh. The qh bits of
// four groups are spread into bytes (a 24-bit multiply), v_perm_b32 interleaves them with the qs bytes into two
// 16-bit indices a dword, and a shift gives each group's LDS address.
#pragma once
#include <stdlib.h>

#include <algorithm>

#include "fast_impl.h"

namespace strata_mv {

constexpr int kWLoads = 8;          // 16-byte loads a lane keeps in flight: an item is at most 8 KB
constexpr int kWaves = 4;           // waves a workgroup
constexpr int kPMaxPairs = 256;     // pairs the persistent kernel holds in LDS (one a thread at set-up)
constexpr int kWaveStage = kWLoads * 64 * 16 + 32;
constexpr int kWorkgroupsPerCU = 3;

// Run n of a row as 16 packed float16 pairs of integers and its scale; IQ3_S through perm-built indices.
template <int KIND>
__device__ __forceinline__ float decode_run(const uint8_t* row, uint32_t n, uint32_t* w, const FastTables<KIND>& t) {
  if constexpr (KIND == K_IQ3_S) {
    const uint8_t* b = row + (n >> 3) * 110;
    const uint32_t ib = n & 7;
    const float scale =
        strata_half_at(b) * (float)(1 + 2 * (((uint32_t)b[106 + (ib >> 1)] >> (4 * (ib & 1))) & 15));
    const uint32_t qs0 = lds_u32(b + 2 + 8 * ib), qs1 = lds_u32(b + 6 + 8 * ib);
    const uint32_t qh = b[66 + ib];
    const uint32_t sg = lds_u32(b + 74 + 4 * ib);
    const uint32_t hb0 = (__builtin_amdgcn_ubfe(qh, 0, 4) * 0x204081u) & 0x01010101u;
    const uint32_t hb1 = (__builtin_amdgcn_ubfe(qh, 4, 4) * 0x204081u) & 0x01010101u;
    const uint32_t i01 = __builtin_amdgcn_perm(hb0, qs0, 0x05010400u), i23 = __builtin_amdgcn_perm(hb0, qs0, 0x07030602u);
    const uint32_t i45 = __builtin_amdgcn_perm(hb1, qs1, 0x05010400u), i67 = __builtin_amdgcn_perm(hb1, qs1, 0x07030602u);
    const uint32_t ix[8] = {i01 & 0xffff, i01 >> 16, i23 & 0xffff, i23 >> 16,
                            i45 & 0xffff, i45 >> 16, i67 & 0xffff, i67 >> 16};
#pragma unroll
    for (int l = 0; l < 8; ++l) {
      const u32x2 g = t.grid[ix[l]];
      const u32x4 m = t.signs[(sg >> (8 * (l >> 1))) & 255];
      w[2 * l] = g[0] ^ m[(l & 1) * 2];
      w[2 * l + 1] = g[1] ^ m[(l & 1) * 2 + 1];
    }
    return scale;
  } else {
    return fast_decode<KIND>(row, n, w, t);
  }
}

// dot16 with two chains, so that consecutive v_dot2 do not wait on each other
__device__ __forceinline__ float dot16x2(const uint32_t* w, const uint32_t* x) {
  float a = 0.0f, b = 0.0f;
#pragma unroll
  for (int i = 0; i < 16; i += 2) {
    a = __builtin_amdgcn_fdot2(__builtin_bit_cast(h2_t, w[i]), __builtin_bit_cast(h2_t, x[i]), a, false);
    b = __builtin_amdgcn_fdot2(__builtin_bit_cast(h2_t, w[i + 1]), __builtin_bit_cast(h2_t, x[i + 1]), b, false);
  }
  return a + b;
}

template <int KIND, bool GLU, int TT, int RPL>
__global__ __launch_bounds__(kThreads, 3) void wave_decode_kernel(MatvecParams p) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  FastTables<KIND>& tab = *reinterpret_cast<FastTables<KIND>*>(smem);
  size_t off = (sizeof(FastTables<KIND>) + 15) & ~(size_t)15;
  uint32_t* idx_l = reinterpret_cast<uint32_t*>(smem + off);  // expert of each pair, bit 31: an earlier pair names it
  off += kPMaxPairs * sizeof(uint32_t);
  int16_t* next_l = reinterpret_cast<int16_t*>(smem + off);  // the next pair naming the same expert, or -1
  off += kPMaxPairs * sizeof(int16_t);
  const int wave = threadIdx.x / 64, lane = threadIdx.x % 64;
  uint8_t* stage = smem + off + (size_t)wave * kWaveStage;

  const int tid = threadIdx.x, nt = blockDim.x;
  const bool expert_mode = p.mode == MODE_EXPERT;
  fast_load_tables<KIND>(tab, tid, nt);
  if (expert_mode) {
    // an id past the stack reads as 0x7fffffff: never bit 31, never equal to a real expert
    const uint32_t e = tid < p.pairs ? p.idx[tid] : 0x7fffffffu;
    const uint32_t ev = e < (uint64_t)p.experts ? e : 0x7fffffffu;
    if (tid < p.pairs) idx_l[tid] = ev;
    __syncthreads();
    bool dup = false;
    int next = -1;
    if (tid < p.pairs && ev != 0x7fffffffu) {  // all lanes read the same entry at a time: LDS broadcasts
      for (int r = 0; r < tid && !dup; ++r) dup = idx_l[r] == ev;
      for (int r = tid + 1; r < p.pairs && next < 0; ++r)
        if (idx_l[r] == ev) next = r;
    }
    __syncthreads();  // every lane has read idx_l before the flags go in
    if (tid < p.pairs) {
      next_l[tid] = (int16_t)next;
      if (dup) idx_l[tid] = ev | 0x80000000u;
    }
  }
  __syncthreads();

  const int L = p.ct;            // lanes to a row
  const int rows_side = 64 / L;  // rows a wave decodes side by side
  const int sub = lane / L, ln = lane % L;
  const int per_mat = p.ntiles, per_pair = p.nz * per_mat;
  const int wave_id = blockIdx.x * kWaves + wave, waves = gridDim.x * kWaves;

  auto valid_from = [&](int it) {
    if (expert_mode)
      while (it < p.items && (idx_l[it / per_pair] & 0x80000000u)) it += waves;
    return it;
  };
  auto locate = [&](int it, const uint8_t*& mat, int& z, int& r0, int& nr, int& pair) {
    pair = it / per_pair;
    const int rem = it % per_pair;
    z = rem / per_mat;
    r0 = (rem % per_mat) * p.rt;
    nr = min(p.rt, p.rows - r0);
    if (expert_mode) {
      const uint32_t e = idx_l[pair] & 0x7fffffffu;
      mat = e < (uint64_t)p.experts ? p.blocks[z] + (int64_t)e * p.mat_bytes : nullptr;
    } else if (p.mode == MODE_PTRS) {
      mat = p.ptrs[pair];
    } else {
      mat = p.blocks[z];
    }
  };

  u32x4 v[kWLoads];
  uintptr_t lo = 0, hi = 0, a0 = 0, a1 = 0;
  int chunks = 0;
  auto issue = [&](int it) {
    const uint8_t* mat;
    int z, r0, nr, pair;
    locate(it, mat, z, r0, nr, pair);
    chunks = 0;
    if (mat == nullptr) return;
    lo = (uintptr_t)(mat + (int64_t)r0 * p.row_bytes);
    hi = lo + (uintptr_t)nr * p.row_bytes;
    a0 = (lo + 15) & ~(uintptr_t)15;
    a1 = hi & ~(uintptr_t)15;
    chunks = a1 > a0 ? (int)((a1 - a0) >> 4) : 0;
#pragma unroll
    for (int i = 0; i < kWLoads; ++i)
      if (lane + i * 64 < chunks) v[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(a0) + lane + i * 64);
  };

  int cur = valid_from(wave_id);
  if (cur >= p.items) return;
  issue(cur);

  // activations every item shares: one token's row for gate/up, or a window of at most TT tokens
  const bool shared_x = !GLU && ((expert_mode && p.share == p.pairs) || (p.mode == MODE_DENSE && p.tokens <= TT));
  uint32_t x[TT][RPL][16];
  auto load_x = [&](int t, int q) {
#pragma unroll
    for (int k = 0; k < RPL; ++k) {
      const int run = ln + k * L;
      if (run < p.runs) fast_load_x<GLU>(p, q, run, x[t][k]);
    }
  };
  if (shared_x) {
    const int nshared = p.mode == MODE_DENSE ? p.tokens : 1;
#pragma unroll
    for (int t = 0; t < TT; ++t)
      if (t < nshared) load_x(t, t);  // window: token t; routed: pair 0, whose x row is the one token's
  }

  for (;;) {
    const uint8_t* mat;
    int z, r0, nr, pair;
    locate(cur, mat, z, r0, nr, pair);
    f16* out = reinterpret_cast<f16*>(p.out[z]);
    const uintptr_t lead = lo & 15;
    if (mat != nullptr) {  // this item's bytes into the wave's stage
      uint8_t* base = stage + lead - lo;
#pragma unroll
      for (int i = 0; i < kWLoads; ++i)
        if (lane + i * 64 < chunks) reinterpret_cast<u32x4*>(base + a0)[lane + i * 64] = v[i];
      if (a0 > a1) {
        for (uintptr_t g = lo + lane; g < hi; g += 64) base[g] = *(const uint8_t*)g;
      } else {
        for (uintptr_t g = lo + lane; g < a0; g += 64) base[g] = *(const uint8_t*)g;
        for (uintptr_t g = a1 + lane; g < hi; g += 64) base[g] = *(const uint8_t*)g;
      }
    }
    __builtin_amdgcn_wave_barrier();  // a wave's LDS operations run in order: its own writes are seen
    const int nxt = valid_from(cur + waves);
    bool issued = false;

    if (mat == nullptr) {  // a pair naming no expert: NaN, nothing read
      for (int r = r0 + lane; r < r0 + nr; r += 64) out[(int64_t)pair * p.rows + r] = (f16)__builtin_nanf("");
    } else {
      const uint8_t* rows0 = stage + lead;
      int member = expert_mode ? pair : 0;  // the next pair (or token) to take
      for (;;) {
        int q[TT];
        int nq = 0;
        if (p.mode == MODE_DENSE) {
          nq = shared_x ? (member == 0 ? p.tokens : 0) : max(0, min(TT, p.tokens - member));
#pragma unroll
          for (int t = 0; t < TT; ++t) q[t] = member + t;
          member += nq;
        } else if (p.mode == MODE_PTRS) {
          nq = member == 0 ? 1 : 0;
          q[0] = pair;
          member = 1;
        } else {
#pragma unroll
          for (int t = 0; t < TT; ++t) {
            q[t] = member;
            if (member >= 0) {
              ++nq;
              member = next_l[member];
            }
          }
        }
        if (nq == 0) break;
        if (!shared_x) {
#pragma unroll
          for (int t = 0; t < TT; ++t)
            if (t < nq) load_x(t, q[t]);
        }
        if (!issued) {  // the next item's loads, in flight while this one computes
          if (nxt < p.items) issue(nxt);
          issued = true;
        }
        for (int rr = 0; rr < nr; rr += rows_side) {
          const int r = rr + sub;
          float s[TT];
#pragma unroll
          for (int t = 0; t < TT; ++t) s[t] = 0.0f;
          if (r < nr) {
#pragma unroll
            for (int k = 0; k < RPL; ++k) {
              const int run = ln + k * L;
              if (run < p.runs) {
                uint32_t w[16];
                const float scale = decode_run<KIND>(rows0 + r * p.row_bytes, (uint32_t)run, w, tab);
#pragma unroll
                for (int t = 0; t < TT; ++t)
                  if (t < nq) s[t] += scale * dot16x2(w, x[t][k]);
              }
            }
          }
#pragma unroll
          for (int t = 0; t < TT; ++t) {
            float v2 = s[t];
            for (int o = L / 2; o >= 1; o /= 2) v2 += __shfl_xor(v2, o, L);
            if (t < nq && ln == 0 && r < nr) out[(int64_t)q[t] * p.rows + r0 + r] = from_f32<f16>(v2);
          }
        }
        if (p.mode == MODE_PTRS || (p.mode == MODE_DENSE && shared_x)) break;
        if (p.mode == MODE_EXPERT && member < 0) break;
      }
    }
    if (!issued && nxt < p.items) issue(nxt);
    __builtin_amdgcn_wave_barrier();  // every lane has read the stage before the next item overwrites it
    cur = nxt;
    if (cur >= p.items) break;
  }
}

// Rows a wave's item holds, at most.
constexpr int kRowsPerItem = 8;

inline int device_cus() {
  static int cus[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cus[dev] == 0) {
    int v = 0;
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v <= 0) v = 256;
    cus[dev] = v;
  }
  return cus[dev];
}

// Lanes to a row and runs a lane: the fewest idle lanes, then the widest rows (at most four runs a lane).
inline int wave_lanes(int runs, int* rpl) {
  int best = 0, best_rpl = 0, best_idle = 1 << 30;
  for (int L : {64, 32, 16}) {
    const int r = (runs + L - 1) / L;
    if (r > 4) continue;
    const int idle = r * L - runs;
    if (idle < best_idle) {
      best_idle = idle;
      best = L;
      best_rpl = r;
    }
  }
  *rpl = best_rpl;
  return best;
}

template <int KIND, bool GLU, int TT, int RPL>
int launch_wave_decode(MatvecParams& p, int grid_y, int grid_z, hipStream_t stream) {
  p.tt = TT;
  p.nz = grid_z;
  const int rows_side = 64 / p.ct;
  int rt = rows_side * std::max(1, kRowsPerItem / rows_side);
  while (rt > rows_side && rt * p.row_bytes + 16 > kWLoads * 64 * 16) rt -= rows_side;
  if (rt * p.row_bytes + 16 > kWLoads * 64 * 16) return STRATA_ERR_SHAPE;
  p.rt = rt;
  p.ntiles = (p.rows + p.rt - 1) / p.rt;
  const int64_t items = (int64_t)grid_y * grid_z * p.ntiles;
  if (items > INT32_MAX) return STRATA_ERR_SHAPE;
  p.items = (int)items;
  const size_t smem = ((sizeof(FastTables<KIND>) + 15) & ~(size_t)15) +
                      kPMaxPairs * (sizeof(uint32_t) + sizeof(int16_t)) + (size_t)kWaves * kWaveStage;
  const int64_t want = (items + kWaves - 1) / kWaves;
  const int grid = (int)std::min<int64_t>(want, (int64_t)kWorkgroupsPerCU * device_cus());
  hipLaunchKernelGGL((wave_decode_kernel<KIND, GLU, TT, RPL>), dim3(grid), dim3(kThreads), smem, stream, p);
  STRATA_CHECK_LAUNCH();
  return STRATA_OK;
}

// Runs a lane (RPL) and tokens a pass (TT, at most 4 / RPL so that the activations fit the registers).
template <int KIND, bool GLU>
int launch_wave_rpl(MatvecParams& p, bool one_token, int grid_y, int grid_z, hipStream_t s) {
  p.runs = p.cols / 32;
  int rpl = 0;
  p.ct = wave_lanes(p.runs, &rpl);
  if (one_token || rpl >= 3) {
    switch (rpl) {
      case 1: return launch_wave_decode<KIND, GLU, 1, 1>(p, grid_y, grid_z, s);
      case 2: return launch_wave_decode<KIND, GLU, 1, 2>(p, grid_y, grid_z, s);
      case 3: return launch_wave_decode<KIND, GLU, 1, 3>(p, grid_y, grid_z, s);
      case 4: return launch_wave_decode<KIND, GLU, 1, 4>(p, grid_y, grid_z, s);
      default: return STRATA_ERR_SHAPE;
    }
  }
  if (rpl == 2) return launch_wave_decode<KIND, GLU, 2, 2>(p, grid_y, grid_z, s);
  return launch_wave_decode<KIND, GLU, 4, 1>(p, grid_y, grid_z, s);
}

}  // namespace strata_mv
