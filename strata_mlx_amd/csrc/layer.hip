// The routed experts of one decode token as one launch: gate and up with the SwiGLU, then down, IQ3_S or Q2_0,
// float16 (strata_mlx/blocks.py:958-986 at one token: the gate and up calls and matvec_glu's down with the
// SwiGLU, :939-955, rounded as _MATVEC_GLU rounds it, :222-236).
//
// As two launches (routed_impl.h) a layer pays two launch boundaries, two prologues (the 64 KB signed codebook
// built in every CU's LDS) and two decode tails, and down's rows are not asked for until gate/up has ended. Here
// one persistent workgroup a CU does both halves. The workgroups of pair p are those with blockIdx % pairs == p:
// at eight pairs, the 32 workgroups of one XCD (the hardware places workgroup i on XCD i % 8), which compute the
// pair's gate/up rows, hand the pair's h over to each other, and compute its down rows. Down's rows are asked for
// as soon as a wave has decoded its gate/up units, so they arrive while the other waves finish and while h is
// handed over.
//
// The handover is through memory, one 64-bit word a row of h: the launch's tag (high 32 bits) and h's float16
// bits (low 16), stored and read with agent-scope relaxed atomics (global_store / global_load with sc1, which are
// coherent across the XCDs' L2s). The tag is the data's own ready flag, so nothing orders one store after another
// and no counter is shared between workgroups. So that the waiting does not flood memory (every thread polling its
// words kept the whole pair's h in flight, 12 KB a workgroup a poll, and the layer took 27 us against 21 as two
// launches), each workgroup also stores a flag with the tag once all its waves have stored their h, and one wave
// polls the pair's flags (a few cache lines) before the words are read; a flag is only a hint, since a word whose
// tag is not yet there is read again. A launch's tag is one more than the last launch's: every
// workgroup keeps its own launch count in the workspace (all of them advance together, since every launch has
// one workgroup a CU and each bumps its own), so the graph that replays this launch with the same arguments
// still tags every launch apart. A word keeps the tag of the launch that last wrote it, so a stale word could
// only pass for a fresh one after 2^32 launches.
//
// Every wait is bounded: a workgroup that polls a flag or a word `spin` times without finding the tag gives up, writes NaN
// for its down rows and sets bit 0 of the workspace's status word (which the caller reads and clears). Every
// workgroup of the grid must be resident at once for the handover to complete; one workgroup a CU and a grid of
// one workgroup a CU make that so on an idle device.
#include "direct_impl.h"

namespace strata_mv {

// Workspace (uint32 words): [0] status (bit 0: a wait gave up), [64, 64 + kLayerMaxGroups) each workgroup's
// launch count, [kLayerFlagsAt, + kLayerMaxGroups) each workgroup's flag (pair-major: pair * slots + slot), from
// byte kLayerWordsAt the tagged words of h, pairs x ffn uint64.
constexpr int kLayerMaxGroups = 1024;
constexpr int kLayerCountAt = 64;
constexpr int kLayerFlagsAt = kLayerCountAt + kLayerMaxGroups;
constexpr int64_t kLayerWordsAt = 16384;
constexpr int kLayerMaxPairs = 16;

struct LayerParams {
  const uint8_t* gate;
  const uint8_t* up;
  const uint8_t* down;
  const uint32_t* idx;  // the expert of each pair
  const u32x4* x;       // the token: 4096 float16 as 512 pieces of 16 bytes
  f16* h;               // (pairs, ffn) silu(gate . x) * (up . x), or null
  f16* y;               // (pairs, 4096) down . h
  uint32_t* ws;
  int64_t gu_mat_bytes, dn_mat_bytes;
  uint32_t experts;
  int ffn, gu_row_bytes, dn_rows, dn_row_bytes, pairs;
  int slots;  // workgroups a pair; workgroups from pairs * slots on only advance their launch count
  int spin;   // polls of a word before a workgroup gives up
};

__device__ __forceinline__ uint64_t* layer_words(uint32_t* ws) {
  return reinterpret_cast<uint64_t*>(reinterpret_cast<uint8_t*>(ws) + kLayerWordsAt);
}

// KIND: IQ3_S or Q2_0. UPW: gate/up units a wave (unit: row r of gate and of up). S: down's run pairs a lane
// (8 lanes a row: ffn = 512 S). DUPW: down units a wave (8 rows each).
template <int KIND, int UPW, int S, int DUPW>
__global__ __launch_bounds__(kGluThreads, 1) void routed_layer_kernel(LayerParams p) {
  typedef Routed<KIND> R;
  typedef typename R::Fields Fields;
  constexpr int kBuffers = UPW < R::kBuffers ? UPW : R::kBuffers;  // units whose rows are in registers at once
  constexpr int kTabBytes = (8 * R::kEntries + 15) / 16 * 16;
  constexpr int kHPieces = 8 * 8 * S;  // h as down's token: 16-byte pieces
  __shared__ __attribute__((aligned(16))) uint8_t lds[kTabBytes + 16 * 512 + 16 * kHPieces + 16];
  // down units a wave may claim (twice its share where the registers hold them: rows of 1536 inputs, one unit a
  // wave), and a workgroup's
  constexpr int kClaim = S == 3 && DUPW == 1 ? 2 : DUPW, kUnits = kGluWaves * DUPW;
  u32x2* const tab = reinterpret_cast<u32x2*>(lds);
  u32x4* const xs = reinterpret_cast<u32x4*>(lds + kTabBytes);
  u32x4* const hs = reinterpret_cast<u32x4*>(lds + kTabBytes + 16 * 512);
  // the workgroup's words: whether a wait gave up, waves whose gate/up loads are all out, down units claimed, and the
  // first wave that claimed none
  uint32_t* const gave_up = reinterpret_cast<uint32_t*>(lds + kTabBytes + 16 * 512 + 16 * kHPieces);
  uint32_t* const issued = gave_up + 1;
  uint32_t* const claimed = gave_up + 2;
  uint32_t* const poller = gave_up + 3;
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int group = blockIdx.x;
  uint32_t* const count = p.ws + kLayerCountAt + group;
  const uint32_t epoch = __hip_atomic_load(count, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1;
  if (group >= p.pairs * p.slots) {  // no pair: only the launch count advances
    if (tid == 0) __hip_atomic_store(count, epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return;
  }
  const int pair = group % p.pairs, slot = group / p.pairs;
  const int q = slot * kGluWaves + wave;  // the wave's index among its pair's waves

  // what the workgroup shares, asked for first: the codebook entry this thread expands and a piece of the token
  const uint64_t entry = R::fetch(tid);
  const int c = min(tid, 511);  // threads past the token's pieces write one again
  const u32x4 xpiece = p.x[c];
  const uint32_t e = p.idx[pair];
  const bool bad = e >= p.experts;  // a pair naming no expert reads expert 0's rows and writes NaN
  const int64_t expert = bad ? 0 : (int64_t)e;
  R::fill(tab, tid, entry);
  xs[x_piece_slot(c)] = xpiece;
  if (tid == 0) {
    *gave_up = 0;
    *issued = 0;
    *claimed = 0;
    *poller = kGluWaves;
  }
  __syncthreads();
  uint32_t x[32];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int r = run_of<KIND>(lane, h);
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const u32x4 piece = xs[x_piece_slot(4 * r + v)];
#pragma unroll
      for (int i = 0; i < 4; ++i) x[16 * h + 4 * v + i] = piece[i];
    }
  }

  // gate/up: the wave's units are rows q * UPW .. q * UPW + UPW - 1 of its pair
  int row[UPW];
  bool live[UPW];
#pragma unroll
  for (int k = 0; k < UPW; ++k) {
    row[k] = q * UPW + k;
    live[k] = row[k] < p.ffn;
    row[k] = live[k] ? row[k] : p.ffn - 1;  // past the last row: the last row again, nothing written
  }
  const uint8_t* const gate = p.gate + expert * p.gu_mat_bytes;
  const uint8_t* const up = p.up + expert * p.gu_mat_bytes;
  auto issue = [&](int k, Fields(&f)[2]) {
    const int64_t off = (int64_t)row[k] * p.gu_row_bytes;
    R::load(gate + off, lane, f[0]);
    R::load(up + off, lane, f[1]);
    asm volatile("" ::: "memory");  // the units' loads go out in unit order
  };
  Fields f[kBuffers][2];
#pragma unroll
  for (int k = 0; k < kBuffers; ++k) issue(k, f[k]);
  if (UPW <= kBuffers && lane == 0) atomicAdd(issued, 1u);  // this wave's gate/up loads are all out
  float xsum[R::kPrepSums + 1];
  R::prep_x(x, xsum);
  float gv = 0.0f, uv = 0.0f;  // lane k: unit k's two totals
#pragma unroll
  for (int k = 0; k < UPW; ++k) {
    float g, u;
    glu_unit<KIND>(f[k % kBuffers], lane, x, x, xsum, xsum, tab, g, u);
    if (k + kBuffers < UPW) {
      issue(k + kBuffers, f[k % kBuffers]);
      if (k + kBuffers == UPW - 1 && lane == 0) atomicAdd(issued, 1u);
    }
    gv = lane == k ? g : gv;
    uv = lane == k ? u : uv;
  }

  // lane k hands over unit k's h: silu(gate) * up as mlx-lm rounds it, tagged with this launch
  uint64_t* const words = layer_words(p.ws) + (int64_t)pair * p.ffn;
  {
    bool w_live = false;
    int w_row = 0;
#pragma unroll
    for (int k = 0; k < UPW; ++k) {
      if (lane == k) {
        w_live = live[k];
        w_row = row[k];
      }
    }
    if (lane < UPW && w_live) {
      f16 gq = from_f32<f16>(gv), uq = from_f32<f16>(uv), hq;
      if (bad) {
        hq = (f16)__builtin_nanf("");
      } else {
        hq = from_f32<f16>(swiglu_rounded<f16>(gq, uq));
      }
      const uint64_t word = ((uint64_t)epoch << 32) | (uint64_t)__builtin_bit_cast(uint16_t, hq);
      __hip_atomic_store(words + w_row, word, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (p.h != nullptr) p.h[(int64_t)pair * p.ffn + w_row] = hq;
    }
  }

  // Down's rows. The workgroup's units (8 rows each) go to the waves that finish gate/up first, up to kClaim a wave,
  // so that the rows of the last waves' units are not asked for last; and none before every wave's gate/up rows
  // are asked for (down's rows would otherwise go out ahead of them). 8 lanes a row, lane m its run pairs m,
  // m + 8, ... A wave that claims nothing has no loads in flight at the handover: the first such wave polls.
  {
    int n = 0;
    while (__hip_atomic_load(issued, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) < (uint32_t)kGluWaves &&
           ++n < (1 << 22))
      __builtin_amdgcn_s_sleep(1);
  }
  const int m = lane & 7, sub = lane >> 3;
  const uint8_t* const dmat = p.down + expert * p.dn_mat_bytes;
  uint32_t base = 0;
  if (lane == 0) base = atomicAdd(claimed, (uint32_t)kClaim);
  base = __builtin_amdgcn_readfirstlane(base);
  if (base >= (uint32_t)kUnits && lane == 0) atomicMin(poller, (uint32_t)wave);
  int r0[kClaim];
  bool dl[kClaim];
  Fields fd[kClaim][S];
#pragma unroll
  for (int k = 0; k < kClaim; ++k) {
    dl[k] = base + k < (uint32_t)kUnits;
    r0[k] = (slot * kUnits + (int)base + k) * 8;
    if (dl[k]) {
      const int rl = min(r0[k] + sub, p.dn_rows - 1);  // rows past the matrix read its last row, and write nothing
      const uint8_t* rowp = dmat + (int64_t)rl * p.dn_row_bytes;
#pragma unroll
      for (int st = 0; st < S; ++st) R::load(rowp, 8 * st + m, fd[k][st]);
    }
    asm volatile("" ::: "memory");
  }

  // every wave's h is out: the workgroup's flag says so (a hint: the tags decide). One wave then waits for the flags
  // of the pair's other workgroups, a few cache lines a poll, before the words themselves are read.
  __syncthreads();
  uint32_t* const flags = p.ws + kLayerFlagsAt + pair * p.slots;
  if (tid == 0) __hip_atomic_store(flags + slot, epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const uint32_t pw = *poller;
  if ((uint32_t)wave == (pw < (uint32_t)kGluWaves ? pw : 0u)) {
    bool failed = false;
    for (int s0 = 0; s0 < p.slots; s0 += 64) {
      if (s0 + lane < p.slots) {
        int n = 0;
        while (__hip_atomic_load(flags + s0 + lane, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != epoch) {
          if (++n >= p.spin) {
            failed = true;
            break;
          }
          __builtin_amdgcn_s_sleep(2);
        }
      }
    }
    if (failed) atomicOr(gave_up, 1u);
  }
  __syncthreads();
  if (*gave_up == 0) {
    // the pair's h: thread t takes rows 2 t and 2 t + 1 into LDS as down's token
    bool failed = false;
    for (int t = tid; 2 * t < p.ffn; t += kGluThreads) {
      uint64_t a = 0, b = 0;
      int n = 0;
      for (;;) {
        a = __hip_atomic_load(words + 2 * t, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        b = __hip_atomic_load(words + 2 * t + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if ((uint32_t)(a >> 32) == epoch && (uint32_t)(b >> 32) == epoch) break;
        if (++n >= p.spin) {
          failed = true;
          break;
        }
        __builtin_amdgcn_s_sleep(2);
      }
      const int pc = t >> 2;  // the 16-byte piece of rows 2 t, 2 t + 1
      uint32_t* dst = reinterpret_cast<uint32_t*>(hs + glu_x_slot(pc >> 3, pc & 7)) + (t & 3);
      *dst = (uint32_t)(a & 0xFFFFu) | ((uint32_t)(b & 0xFFFFu) << 16);
    }
    if (failed) atomicOr(gave_up, 1u);
  }
  __syncthreads();
  const bool lost = *gave_up != 0;
  if (lost && tid == 0) __hip_atomic_fetch_or(p.ws, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);

  // down: each claimed unit's 8 rows against the pair's h
#pragma unroll
  for (int k = 0; k < kClaim; ++k) {
    if (!dl[k]) continue;
    float acc = 0.0f;
#pragma unroll
    for (int st = 0; st < S; ++st) {
      opaque(fd[k][st]);
      const int j = 8 * st + m;
      uint32_t hx[32];
#pragma unroll
      for (int v = 0; v < 8; ++v) {
        const u32x4 piece = hs[glu_x_slot(j, v)];
#pragma unroll
        for (int i = 0; i < 4; ++i) hx[4 * v + i] = piece[i];
      }
      acc += R::pair_sum_lds(fd[k][st], j, hx, nullptr, tab);
    }
    acc += lanes_apart(acc, 1);
    acc += lanes_apart(acc, 2);
    acc += lanes_apart(acc, 4);
    const int r = r0[k] + sub;
    if (m == 0 && r < p.dn_rows)
      p.y[(int64_t)pair * p.dn_rows + r] = bad || lost ? (f16)__builtin_nanf("") : from_f32<f16>(acc);
  }
  if (tid == 0) __hip_atomic_store(count, epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <int KIND, int S, int DUPW>
int launch_layer_u(LayerParams& p, int upw, int groups, hipStream_t s) {
  const dim3 grid(groups), block(kGluThreads);
  switch (upw) {
    case 1: hipLaunchKernelGGL((routed_layer_kernel<KIND, 1, S, DUPW>), grid, block, 0, s, p); break;
    case 3: hipLaunchKernelGGL((routed_layer_kernel<KIND, 3, S, DUPW>), grid, block, 0, s, p); break;
    case 4: hipLaunchKernelGGL((routed_layer_kernel<KIND, 4, S, DUPW>), grid, block, 0, s, p); break;
    case 6: hipLaunchKernelGGL((routed_layer_kernel<KIND, 6, S, DUPW>), grid, block, 0, s, p); break;
    default: return STRATA_ERR_SHAPE;
  }
  STRATA_CHECK_LAUNCH();
  return STRATA_OK;
}

template <int KIND>
int launch_layer(LayerParams& p, hipStream_t s) {
  const int groups = device_cus();
  if (groups > kLayerMaxGroups || p.pairs > groups) return STRATA_ERR_SHAPE;
  p.slots = groups / p.pairs;
  const int waves = p.slots * kGluWaves;  // a pair's waves
  const int need = (p.ffn + waves - 1) / waves;
  int upw = 0;
  for (int f : {1, 3, 4, 6})  // IQ3_S at two units a wave spills registers (routed_impl.h)
    if (!upw && f >= need) upw = f;
  const int dneed = ((p.dn_rows + 7) / 8 + waves - 1) / waves;
  if (!upw || dneed > 2) return STRATA_ERR_SHAPE;
  if (p.ffn == 1536)
    return dneed == 1 ? launch_layer_u<KIND, 3, 1>(p, upw, groups, s) : launch_layer_u<KIND, 3, 2>(p, upw, groups, s);
  // rows of 2560 inputs at two down units a wave spill registers: those go to the two launches
  return dneed == 1 ? launch_layer_u<KIND, 5, 1>(p, upw, groups, s) : STRATA_ERR_SHAPE;
}

}  // namespace strata_mv

using namespace strata_mv;

extern "C" {

int64_t strata_expert_layer_workspace(int64_t pairs, int64_t ffn) {
  if (pairs < 0 || ffn < 0 || pairs > kLayerMaxPairs || ffn > 2560) return -1;
  return kLayerWordsAt + 8 * pairs * ffn;
}

int strata_expert_layer(int kind, const void* gate_blocks, const void* up_blocks, const void* down_blocks,
                        int64_t experts, int64_t hidden, int64_t ffn, const uint32_t* idx, int64_t pairs,
                        const void* x, int x_dtype, void* out_h, void* out, void* workspace, int64_t spin,
                        void* stream) {
  if (kind != K_IQ3_S && kind != K_Q2_0) return STRATA_ERR_KIND;
  if (x_dtype != DT_F16) return STRATA_ERR_DTYPE;
  if (hidden != 4096 || (ffn != 1536 && ffn != 2560)) return STRATA_ERR_SHAPE;
  if (pairs < 1 || pairs > kLayerMaxPairs || experts < 1 || experts > INT32_MAX || spin < 1 || spin > INT32_MAX)
    return STRATA_ERR_ARG;
  if (!gate_blocks || !up_blocks || !down_blocks || !idx || !x || !out || !workspace) return STRATA_ERR_ARG;
  int per = 0, bb = 0;
  strata_kind_info(kind, &per, &bb);
  LayerParams p = {};
  p.gate = (const uint8_t*)gate_blocks;
  p.up = (const uint8_t*)up_blocks;
  p.down = (const uint8_t*)down_blocks;
  p.idx = idx;
  p.x = (const u32x4*)x;
  p.h = (f16*)out_h;
  p.y = (f16*)out;
  p.ws = (uint32_t*)workspace;
  p.gu_row_bytes = (int)(hidden / per * bb);
  p.dn_row_bytes = (int)(ffn / per * bb);
  p.gu_mat_bytes = ffn * (int64_t)p.gu_row_bytes;
  p.dn_mat_bytes = hidden * (int64_t)p.dn_row_bytes;
  p.experts = (uint32_t)experts;
  p.ffn = (int)ffn;
  p.dn_rows = (int)hidden;
  p.pairs = (int)pairs;
  p.spin = (int)spin;
  return kind == K_IQ3_S ? launch_layer<K_IQ3_S>(p, (hipStream_t)stream)
                         : launch_layer<K_Q2_0>(p, (hipStream_t)stream);
}

}  // extern "C"
