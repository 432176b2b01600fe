// Kernel templates of the matvec family; instantiated once per block type by matvec_kind.hip.
#pragma once
// Dequant and the bandwidth-bound matvec family on the file's own blocks (no MFMA).
//
// Matvec layout. A workgroup takes `rt` consecutive rows of one matrix (a "row tile"):
//   1. it stages the tile's bytes from HBM into LDS with 16-byte loads, coalesced over the whole
//      tile (the rows of a matrix are contiguous in the file's layout);
//   2. thread (c, l) decodes run c (columns 32c .. 32c+31) of rows l, l + rs, ... from LDS and
//      multiplies them by the activations of that run, which it holds in registers for the whole
//      tile: a thread always works on the same 32 columns;
//   3. the partial sums of a row (one per run) are added in LDS, eight lanes to a row, and written
//      once in the output dtype.
// The routed form (strata_mlx/blocks.py:196-220) gives a workgroup one pair; a pair whose expert an
// earlier pair also names leaves the work to that one, which multiplies the expert's rows by the
// activations of every pair naming it: an expert's bytes are read once per call.
#include <type_traits>

#include "decode.h"

namespace strata_mv {

constexpr int kThreads = 256;
constexpr int kRowsPerLane = 8;
constexpr int kMaxQueue = 64;  // pairs sharing one expert handled by one workgroup, per pass

enum MatvecMode : int { MODE_EXPERT = 0, MODE_PTRS = 1, MODE_DENSE = 2 };

struct MatvecParams {
  const uint8_t* blocks[2];    // expert / dense mode: the stacks (z selects one)
  void* out[2];
  const uint8_t* const* ptrs;  // ptrs mode: a matrix per pair
  const uint32_t* idx;         // expert mode: expert of each pair
  const uint32_t* row_ids;     // dense mode: rows to compute, or null for all
  const void* x;               // activations, or gate in GLU mode
  const void* up;              // GLU mode
  void* glu_out;               // paired gate/up mode: silu(gate) * up, rounded as mlx-lm rounds it
  int64_t mat_bytes;           // rows_in_matrix * row_bytes
  int64_t experts;             // expert mode: matrices in the stack
  int src_rows;                // rows of the matrix (row_ids must be below it)
  int rows;                    // output rows (n_ids when row_ids is set)
  int cols, row_bytes, runs;
  int pairs, share, tokens;
  int ct, rs, rt;              // column threads (= runs), row lanes, rows per tile
  int tt;                      // tokens a pass holds in registers (<= TT)
  int nz, ntiles, items;       // persistent decode: stacks, row tiles per matrix, work items
  int mode;
  int stage_bytes;             // LDS bytes for the staged rows
  // a shared expert in the routed gate/up launch (one token): its Q4_K gate and up (shared_rows x cols) and its h
  const uint8_t* shared[2];
  void* shared_out;
  void* shared_gu[2];  // the shared expert's gate . x and up . x, or null
  const void* shared_x;  // the shared expert's token in the routed down launch (its h)
  int shared_rows, shared_row_bytes;
  // the choice of experts made in the routed gate/up launch (one token): the router's logits (route_rows float32,
  // the experts' route_experts first), the choice out (idx, weights) and the rows past the experts' as float16
  const float* route_logits;
  uint32_t* route_idx;
  float* route_w;
  void* route_extra;
  int route_rows, route_experts;
};

// Copy [src, src + len) to LDS at dst + (src & 15), 16-byte loads for the aligned middle.
__device__ __forceinline__ void stage_bytes(uint8_t* dst, const uint8_t* src, int len, int tid, int nt) {
  uintptr_t lo = (uintptr_t)src, hi = lo + (uintptr_t)len;
  uintptr_t a0 = (lo + 15) & ~(uintptr_t)15, a1 = hi & ~(uintptr_t)15;
  uint8_t* base = dst + (lo & 15) - lo;  // LDS address of global byte g is base + g
  if (a0 > a1) {                          // shorter than one aligned chunk
    for (uintptr_t g = lo + tid; g < hi; g += nt) base[g] = *(const uint8_t*)g;
    return;
  }
  for (uintptr_t g = lo + tid; g < a0; g += nt) base[g] = *(const uint8_t*)g;
  for (uintptr_t g = a1 + tid; g < hi; g += nt) base[g] = *(const uint8_t*)g;
  int chunks = (int)((a1 - a0) >> 4);
  const u32x4* s4 = (const u32x4*)a0;
  u32x4* d4 = (u32x4*)(base + a0);
  int i = tid;
  for (; i + 3 * nt < chunks; i += 4 * nt) {  // four loads in flight per thread
    u32x4 v0 = __builtin_nontemporal_load(s4 + i);
    u32x4 v1 = __builtin_nontemporal_load(s4 + i + nt);
    u32x4 v2 = __builtin_nontemporal_load(s4 + i + 2 * nt);
    u32x4 v3 = __builtin_nontemporal_load(s4 + i + 3 * nt);
    d4[i] = v0;
    d4[i + nt] = v1;
    d4[i + 2 * nt] = v2;
    d4[i + 3 * nt] = v3;
  }
  for (; i < chunks; i += nt) d4[i] = __builtin_nontemporal_load(s4 + i);
}

// The next pairs naming `expert` from `scan` on, at most tt of them, in pair order, into queue; returns how many
// and moves `scan` past the last one taken. Every thread of the workgroup calls it: a window of blockDim.x pairs
// at a time, one ballot a wave, the waves' counts added in LDS (wcount: blockDim.x / 64 + 1 ints).
__device__ __forceinline__ int next_pairs(const uint32_t* idx, int pairs, uint32_t expert, int tt, int& scan,
                                          uint32_t* queue, int* wcount) {
  const int tid = threadIdx.x, lane = tid % 64, wave = tid / 64, nw = blockDim.x / 64;
  int n = 0;
  while (n < tt && scan < pairs) {
    __syncthreads();  // the last window's counts have been read
    const int q = scan + tid;
    const bool hit = q < pairs && idx[q] == expert;
    const uint64_t m = __ballot(hit);
    if (lane == 0) wcount[wave] = __popcll(m);
    __syncthreads();
    int before = 0, total = 0;
    for (int w = 0; w < nw; ++w) {
      const int c = wcount[w];
      before += w < wave ? c : 0;
      total += c;
    }
    const int rank = n + before + __popcll(m & ((1ull << lane) - 1));
    if (hit && rank < tt) queue[rank] = q;
    if (hit && rank == tt - 1) wcount[nw] = q + 1;
    __syncthreads();
    if (n + total >= tt) {
      scan = wcount[nw];
      n = tt;
    } else {
      scan += blockDim.x;
      n += total;
    }
  }
  __syncthreads();  // the queue is written
  return n;
}

template <typename XT>
__device__ __forceinline__ void load_run(const XT* x, float* v) {
#pragma unroll
  for (int j = 0; j < 32; ++j) v[j] = to_f32(x[j]);
}

// silu(g) * u as mlx-lm rounds it (strata_mlx/blocks.py:230-238): the sigmoid in float32 rounded to
// XT, then g * sig and that times u, each product rounded to XT.
template <typename XT>
__device__ __forceinline__ float swiglu_rounded(XT g, XT u) {
  float gf = to_f32(g);
  float y = 1.0f / (1.0f + expf(fabsf(gf)));
  XT sig = from_f32<XT>(gf < 0.0f ? y : 1.0f - y);
  XT a = from_f32<XT>(gf * to_f32(sig));
  return to_f32(from_f32<XT>(to_f32(a) * to_f32(u)));
}

template <int KIND, typename XT, typename OT, bool GLU, int TT>
__global__ __launch_bounds__(kThreads, 2) void matvec_kernel(MatvecParams p) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  StrataTables& tab = *reinterpret_cast<StrataTables*>(smem);
  uint32_t* queue = reinterpret_cast<uint32_t*>(smem + sizeof(StrataTables));
  int* nqueue = reinterpret_cast<int*>(queue + kMaxQueue);  // also the waves' counts of next_pairs
  uint8_t* stage = smem + sizeof(StrataTables) + (kMaxQueue + kThreads / 64 + 4) * sizeof(uint32_t);
  float* red = reinterpret_cast<float*>(stage + p.stage_bytes);

  const int tid = threadIdx.x, nt = blockDim.x;
  const int z = blockIdx.z;
  const int r0 = blockIdx.x * p.rt;
  const int nr = min(p.rt, p.rows - r0);
  strata_load_tables<KIND>(tab);

  // which matrix, and which pairs (or tokens) multiply it
  const uint8_t* mat;
  uint32_t expert = 0;
  int first = 0;
  if (p.mode == MODE_EXPERT) {
    first = blockIdx.y;
    expert = p.idx[first];
    if (expert >= (uint64_t)p.experts) {  // no such expert: its outputs are NaN, nothing is read
      OT* o = reinterpret_cast<OT*>(p.out[z]) + (int64_t)first * p.rows;
      for (int r = r0 + tid; r < r0 + nr; r += blockDim.x) o[r] = from_f32<OT>(__builtin_nanf(""));
      return;
    }
    mat = p.blocks[z] + (int64_t)expert * p.mat_bytes;
    int dup = 0;  // an earlier pair names this expert and does its work: every thread looks at a share
    for (int q = tid; q < first; q += nt) dup |= p.idx[q] == expert;
    if (__syncthreads_or(dup)) return;
  } else if (p.mode == MODE_PTRS) {
    first = blockIdx.y;
    mat = p.ptrs[first];
  } else {
    mat = p.blocks[z];
  }

  // stage the tile
  if (p.row_ids == nullptr) {
    stage_bytes(stage, mat + (int64_t)r0 * p.row_bytes, nr * p.row_bytes, tid, nt);
  } else {
    const int pitch = (p.row_bytes + 31) & ~15;
    for (int r = 0; r < nr; ++r) {
      const uint32_t id = p.row_ids[r0 + r];  // an id past the matrix reads row 0; its output is NaN
      stage_bytes(stage + r * pitch, mat + (int64_t)(id < (uint32_t)p.src_rows ? id : 0) * p.row_bytes, p.row_bytes,
                  tid, nt);
    }
  }
  const int lead = p.row_ids == nullptr ? (int)((uintptr_t)(mat + (int64_t)r0 * p.row_bytes) & 15) : 0;

  const int c = tid % p.ct, lane_row = tid / p.ct;
  const bool active = lane_row < p.rs;  // threads past ct * rs only help to stage and reduce
  OT* out = reinterpret_cast<OT*>(p.out[z]);

  // the pairs of this expert, in order; processed tt at a time
  int scan = first;  // expert mode: next pair to look at
  int done_tokens = 0;
  for (;;) {
    int nq;
    if (p.mode == MODE_EXPERT) {
      nq = next_pairs(p.idx, p.pairs, expert, p.tt, scan, queue, nqueue);
    } else {
      __syncthreads();  // the last pass has read the queue
      if (tid == 0) {
        int n = 0;
        if (p.mode == MODE_PTRS) {
          if (done_tokens == 0) queue[n++] = first;
        } else {
          for (; done_tokens + n < p.tokens && n < p.tt; ++n) queue[n] = done_tokens + n;
        }
        *nqueue = n;
      }
      __syncthreads();
      nq = *nqueue;
    }
    if (nq == 0) break;
    done_tokens += nq;

    const int stride = p.ct + 1;
    if (active) {
      float xr[TT][32];
#pragma unroll
      for (int t = 0; t < TT; ++t) {
        if (t < nq) {
          const int q = queue[t];
          if constexpr (GLU) {
            const XT* g = reinterpret_cast<const XT*>(p.x) + (int64_t)q * p.cols + 32 * c;
            const XT* u = reinterpret_cast<const XT*>(p.up) + (int64_t)q * p.cols + 32 * c;
#pragma unroll
            for (int j = 0; j < 32; ++j) xr[t][j] = swiglu_rounded<XT>(g[j], u[j]);
          } else {
            const int xrow = p.mode == MODE_DENSE ? q : q / p.share;
            load_run<XT>(reinterpret_cast<const XT*>(p.x) + (int64_t)xrow * p.cols + 32 * c, xr[t]);
          }
        }
      }
      const int pitch = p.row_ids == nullptr ? p.row_bytes : ((p.row_bytes + 31) & ~15);
#pragma unroll 1
      for (int r = lane_row; r < nr; r += p.rs) {  // partial sums straight to LDS: no accumulator array
        const uint8_t* row = stage + lead + r * pitch;
        if (p.row_ids != nullptr) {
          const uint32_t id = p.row_ids[r0 + r];
          row += (uintptr_t)(mat + (int64_t)(id < (uint32_t)p.src_rows ? id : 0) * p.row_bytes) & 15;
        }
        float w[32];
        strata_unpack32<KIND>(row, c, w, tab);
#pragma unroll
        for (int t = 0; t < TT; ++t) {
          if (t < nq) {
            float s = 0.0f;
#pragma unroll
            for (int j = 0; j < 32; ++j) s = __builtin_fmaf(w[j], xr[t][j], s);
            red[(t * p.rt + r) * stride + c] = s;
          }
        }
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
        const float* v = red + (t * p.rt + r) * stride;
        for (int cc = tid % 8; cc < p.ct; cc += 8) s += v[cc];
      }
      s += __shfl_xor(s, 4, 8);
      s += __shfl_xor(s, 2, 8);
      s += __shfl_xor(s, 1, 8);
      if (p.row_ids != nullptr && o < outputs && p.row_ids[r0 + r] >= (uint32_t)p.src_rows) s = __builtin_nanf("");
      if (o < outputs && tid % 8 == 0) out[(int64_t)queue[t] * p.rows + r0 + r] = from_f32<OT>(s);
    }
    if (p.mode == MODE_PTRS) break;
  }
}

template <int KIND, typename OT>
__global__ __launch_bounds__(256) void dequant_kernel(const uint8_t* blocks, int64_t runs_total, int runs_per_row,
                                                      int row_bytes, OT* out) {
  __shared__ StrataTables tab;
  strata_load_tables<KIND>(tab);
  __syncthreads();
  const int64_t u = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (u >= runs_total) return;
  const int64_t r = u / runs_per_row;
  const int n = (int)(u % runs_per_row);
  float w[32];
  strata_unpack32<KIND>(blocks + r * row_bytes, (uint32_t)n, w, tab);
  if constexpr (std::is_same<OT, f16>::value) {  // packed pairs, 16-byte stores (64 bytes a run: aligned)
    u32x4* o4 = reinterpret_cast<u32x4*>(out + u * 32);
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      u32x4 c;
#pragma unroll
      for (int i = 0; i < 4; ++i)
        c[i] = (uint32_t)__builtin_bit_cast(uint16_t, from_f32<f16>(w[8 * v + 2 * i])) |
               ((uint32_t)__builtin_bit_cast(uint16_t, from_f32<f16>(w[8 * v + 2 * i + 1])) << 16);
      o4[v] = c;
    }
  } else {
    OT* o = out + u * 32;
#pragma unroll
    for (int j = 0; j < 32; ++j) o[j] = from_f32<OT>(w[j]);
  }
}

inline int geometry(MatvecParams& p, int tt_max) {
  p.runs = p.cols / 32;
  if (p.runs < 1 || p.runs > kThreads) return STRATA_ERR_SHAPE;
  p.ct = p.runs;
  p.rs = kThreads / p.ct;
  int rpl = kRowsPerLane;  // keep the staged rows within 24 KB and the partial sums within 32 KB
  while (rpl > 1 && (p.rs * rpl * p.row_bytes > 24576 || tt_max * p.rs * rpl * (p.ct + 1) * 4 > 32768)) rpl /= 2;
  p.rt = p.rs * rpl;
  p.tt = tt_max;
  const int pitch = p.row_ids ? ((p.row_bytes + 31) & ~15) : p.row_bytes;
  p.stage_bytes = ((p.rt * pitch + 32) + 15) & ~15;
  return STRATA_OK;
}

// Tokens a pass holds in registers: 4 for 16-bit activations, 2 for float32, 1 for the ptrs mode.
inline int tokens_per_pass(int mode, int dtype) { return mode == MODE_PTRS ? 1 : (dtype == DT_F32 ? 2 : 4); }

template <int KIND, typename XT, typename OT, bool GLU, int TT>
int launch_matvec(MatvecParams& p, int grid_y, int grid_z, hipStream_t stream) {
  int rc = geometry(p, TT);
  if (rc) return rc;
  size_t smem = sizeof(StrataTables) + (kMaxQueue + kThreads / 64 + 4) * sizeof(uint32_t) + p.stage_bytes +
                (size_t)TT * p.rt * (p.ct + 1) * sizeof(float);
  dim3 grid((p.rows + p.rt - 1) / p.rt, grid_y, grid_z);
  hipLaunchKernelGGL((matvec_kernel<KIND, XT, OT, GLU, TT>), grid, dim3(kThreads), smem, stream, p);
  STRATA_CHECK_LAUNCH();
  return STRATA_OK;
}

// Every instance one block type needs: x/out dtypes, the SwiGLU form, the tokens per pass.
template <int KIND>
int launch_matvec_kind(MatvecParams& p, int x_dtype, int out_dtype, bool glu, int grid_y, int grid_z,
                       hipStream_t s) {
  const int tt = tokens_per_pass(p.mode, x_dtype);
  if (x_dtype == DT_F32) {
    if (out_dtype != DT_F32) return STRATA_ERR_DTYPE;
    if (tt == 1) return glu ? STRATA_ERR_ARG : launch_matvec<KIND, float, float, false, 1>(p, grid_y, grid_z, s);
    return glu ? launch_matvec<KIND, float, float, true, 2>(p, grid_y, grid_z, s)
               : launch_matvec<KIND, float, float, false, 2>(p, grid_y, grid_z, s);
  }
  auto run16 = [&](auto* tp) -> int {
    using T = std::remove_pointer_t<decltype(tp)>;
    if (tt == 1) {
      if (glu || out_dtype != x_dtype) return STRATA_ERR_ARG;
      return launch_matvec<KIND, T, T, false, 1>(p, grid_y, grid_z, s);
    }
    if (glu) return out_dtype == x_dtype ? launch_matvec<KIND, T, T, true, 4>(p, grid_y, grid_z, s) : STRATA_ERR_DTYPE;
    if (out_dtype == DT_F32) return launch_matvec<KIND, T, float, false, 4>(p, grid_y, grid_z, s);
    if (out_dtype != x_dtype) return STRATA_ERR_DTYPE;
    return launch_matvec<KIND, T, T, false, 4>(p, grid_y, grid_z, s);
  };
  if (x_dtype == DT_F16) return run16((f16*)nullptr);
  if (x_dtype == DT_BF16) return run16((bf16_t*)nullptr);
  return STRATA_ERR_DTYPE;
}

template <int KIND>
int launch_dequant_kind(const uint8_t* blocks, int64_t runs_total, int runs_per_row, int row_bytes, void* out,
                        int out_dtype, hipStream_t s) {
  const int64_t grid = (runs_total + 255) / 256;
  if (out_dtype == DT_F32)
    hipLaunchKernelGGL((dequant_kernel<KIND, float>), dim3(grid), dim3(256), 0, s, blocks, runs_total, runs_per_row,
                       row_bytes, (float*)out);
  else if (out_dtype == DT_F16)
    hipLaunchKernelGGL((dequant_kernel<KIND, f16>), dim3(grid), dim3(256), 0, s, blocks, runs_total, runs_per_row,
                       row_bytes, (f16*)out);
  else
    return STRATA_ERR_DTYPE;
  STRATA_CHECK_LAUNCH();
  return STRATA_OK;
}

}  // namespace strata_mv
