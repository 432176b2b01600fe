// A prompt's (token, expert) pairs laid out in tiles of `tile` slots, each tile one expert's, on the GPU.
//
// The reference works this out with MLX operations on the GPU so the host never waits for the router
// (strata_mlx/blocks.py:657-681): an argsort by expert, per-expert counts, cumulative sums and scatters.
// Here it is a counting sort in three kernels over blocks of 256 pairs, stable so that an expert's slots
// go in pair order:
//   count  each block counts its pairs per expert                       blk[b][e]
//   scan   per expert, the blocks' exclusive prefix (blk becomes offsets); per-expert tiles, their
//          prefix over experts (the expert's first tile), tile_expert, and every slot made empty
//   place  each pair's rank among its block's pairs of the same expert (wave ballots, then the waves
//          before it), plus its block's offset: the slot; where, token and slot_pair written
// The tile count is pairs / tile + min(experts, pairs) whatever the routing, as the reference's.
#include <atomic>

#include "common.h"

namespace {

constexpr int kBlock = 256;  // pairs per block of the count and place kernels
constexpr uint32_t kNone = 0xffffffffu;

__global__ __launch_bounds__(kBlock) void route_count(const uint32_t* idx, int pairs, int experts, uint32_t* blk) {
  extern __shared__ uint32_t cnt[];  // [experts]
  for (int e = threadIdx.x; e < experts; e += kBlock) cnt[e] = 0;
  __syncthreads();
  const int p = blockIdx.x * kBlock + threadIdx.x;
  if (p < pairs) {
    const uint32_t e = idx[p];
    if (e < (uint32_t)experts) atomicAdd(&cnt[e], 1u);
  }
  __syncthreads();
  uint32_t* row = blk + (int64_t)blockIdx.x * experts;
  for (int e = threadIdx.x; e < experts; e += kBlock) row[e] = cnt[e];
}

// One workgroup of 1024 threads.
__global__ __launch_bounds__(1024) void route_scan(uint32_t* blk, int nblocks, int experts, int tile, int n_tiles,
                                                  uint32_t* first_tile, uint32_t* tile_expert, uint32_t* token,
                                                  uint32_t* slot_pair) {
  extern __shared__ uint32_t sh[];  // tiles per expert, then their scan: [experts + 1]
  __shared__ uint32_t wsum[1024 / 64];
  const int tid = threadIdx.x, nt = blockDim.x, lane = tid & 63, wave = tid >> 6;
  for (int e = tid; e < experts; e += nt) {
    // the expert's count in each block of pairs, 16 blocks' loads at a time, then their running sums stored back
    uint32_t run = 0;
    for (int b0 = 0; b0 < nblocks; b0 += 16) {
      uint32_t v[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) v[i] = b0 + i < nblocks ? blk[(int64_t)(b0 + i) * experts + e] : 0u;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        if (b0 + i < nblocks) blk[(int64_t)(b0 + i) * experts + e] = run;
        run += v[i];
      }
    }
    sh[e] = (run + tile - 1) / tile;
  }
  __syncthreads();
  if (experts <= nt) {  // exclusive scan of the tile counts over the workgroup: a wave's, then the waves' totals
    const uint32_t own = tid < experts ? sh[tid] : 0u;
    uint32_t v = own;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const uint32_t t = (uint32_t)__shfl_up((int)v, d);
      if (lane >= d) v += t;
    }
    if (lane == 63) wsum[wave] = v;
    __syncthreads();
    uint32_t before = 0;
    for (int w = 0; w < wave; ++w) before += wsum[w];
    uint32_t total = 0;
    for (int w = 0; w < nt / 64; ++w) total += wsum[w];
    __syncthreads();  // every thread has read its count
    if (tid < experts) sh[tid] = before + v - own;
    if (tid == 0) sh[experts] = total;
  } else if (tid == 0) {  // more experts than threads: one thread's scan
    uint32_t run = 0;
    for (int e = 0; e < experts; ++e) {
      const uint32_t v = sh[e];
      sh[e] = run;
      run += v;
    }
    sh[experts] = run;
  }
  __syncthreads();
  for (int e = tid; e < experts; e += nt) {
    first_tile[e] = sh[e];
    for (uint32_t t = sh[e]; t < sh[e + 1]; ++t) tile_expert[t] = (uint32_t)e;
  }
  for (int t = (int)sh[experts] + tid; t < n_tiles; t += nt) tile_expert[t] = (uint32_t)experts;
  const int64_t slots = (int64_t)n_tiles * tile;
  for (int64_t s = tid; s < slots; s += nt) {
    token[s] = 0;
    if (slot_pair) slot_pair[s] = kNone;
  }
}

__global__ __launch_bounds__(kBlock) void route_place(const uint32_t* idx, int pairs, int k, int experts, int tile,
                                                      const uint32_t* blk, const uint32_t* first_tile,
                                                      uint32_t* token, uint32_t* where, uint32_t* slot_pair) {
  extern __shared__ uint32_t wcnt[];  // [4 waves][experts]: pairs of each expert in each wave
  const int tid = threadIdx.x, wave = tid / 64, lane = tid % 64;
  for (int i = tid; i < 4 * experts; i += kBlock) wcnt[i] = 0;
  __syncthreads();
  const int p = blockIdx.x * kBlock + tid;
  const bool valid = p < pairs && idx[p] < (uint32_t)experts;
  const uint32_t e = valid ? idx[p] : kNone;
  // the lanes of this wave with the same expert: one ballot per distinct expert in the wave
  uint64_t remaining = __ballot(valid);
  uint64_t mine = 0;
  while (remaining) {
    const int leader = __ffsll((unsigned long long)remaining) - 1;
    const uint32_t le = __shfl(e, leader);
    const uint64_t same = __ballot(valid && e == le);
    if (valid && e == le) mine = same;
    if (lane == leader) wcnt[wave * experts + le] = (uint32_t)__popcll(same);
    remaining &= ~same;
  }
  __syncthreads();
  if (p < pairs) {
    if (!valid) {
      where[p] = kNone;
      return;
    }
    uint32_t rank = blk[(int64_t)blockIdx.x * experts + e] + (uint32_t)__popcll(mine & ((1ull << lane) - 1));
    for (int w = 0; w < wave; ++w) rank += wcnt[w * experts + e];
    const uint32_t slot = first_tile[e] * tile + rank;
    where[p] = slot;
    token[slot] = (uint32_t)(p / k);
    if (slot_pair) slot_pair[slot] = (uint32_t)p;
  }
}

// The workspace of strata_route_tiles_noalloc: the library's own device memory, sized for its largest call. Every
// word the kernels read is written by the same call first (the counts by route_count, the first tiles by
// route_scan), so the array needs no clearing between calls; calls that overlap on one GPU share it and race.
constexpr int64_t kScratchPairs = 65536;  // pairs a call takes at most (8192 tokens x top-8)
constexpr int64_t kScratchExperts = 1024;
constexpr int64_t kScratchWords = ((kScratchPairs + kBlock - 1) / kBlock) * kScratchExperts + kScratchExperts + 64;
__device__ __align__(256) uint32_t scratch[kScratchWords];

// scratch's device address on each device, looked up once per device with that device current (in host code the
// array's name stands in for it and is not a device address)
constexpr int kMaxDevices = 64;
std::atomic<void*> scratch_ptr[kMaxDevices];

void* device_scratch() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return nullptr;
  void* p = scratch_ptr[dev].load(std::memory_order_acquire);
  if (p == nullptr) {
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || p == nullptr) return nullptr;
    scratch_ptr[dev].store(p, std::memory_order_release);
  }
  return p;
}

}  // namespace

extern "C" {

int64_t strata_route_tiles_max(int64_t pairs, int64_t experts, int64_t tile) {
  if (pairs < 0 || experts < 0 || tile <= 0) return 0;
  return pairs / tile + (experts < pairs ? experts : pairs);
}

int64_t strata_route_tiles_workspace(int64_t pairs, int64_t experts) {
  if (pairs < 0 || experts < 0) return 0;
  const int64_t nblocks = (pairs + kBlock - 1) / kBlock;
  return (nblocks * experts + experts + 64) * (int64_t)sizeof(uint32_t);
}

int strata_route_tiles(const uint32_t* idx, int64_t pairs, int64_t k, int64_t experts, int64_t tile,
                       uint32_t* tile_expert, uint32_t* token, uint32_t* where, uint32_t* slot_pair, void* workspace,
                       void* stream) {
  if (pairs < 0 || k < 1 || experts < 1 || tile < 1 || tile > 1024) return STRATA_ERR_ARG;
  if (experts > 2048 || pairs > (1 << 24)) return STRATA_ERR_SHAPE;  // the place kernel holds 4 x experts counts in LDS
  const int64_t n_tiles = strata_route_tiles_max(pairs, experts, tile);
  if (n_tiles == 0) return STRATA_OK;
  if (!tile_expert || !token || !workspace || (pairs > 0 && (!idx || !where))) return STRATA_ERR_ARG;
  hipStream_t s = (hipStream_t)stream;
  const int nblocks = (int)((pairs + kBlock - 1) / kBlock);
  uint32_t* blk = (uint32_t*)workspace;
  uint32_t* first_tile = blk + (int64_t)nblocks * experts;
  const size_t lds_e = (size_t)experts * sizeof(uint32_t);
  if (nblocks > 0) {
    hipLaunchKernelGGL(route_count, dim3(nblocks), dim3(kBlock), lds_e, s, idx, (int)pairs, (int)experts, blk);
    STRATA_CHECK_LAUNCH();
  }
  hipLaunchKernelGGL(route_scan, dim3(1), dim3(1024), lds_e + sizeof(uint32_t), s, blk, nblocks, (int)experts,
                     (int)tile, (int)n_tiles, first_tile, tile_expert, token, slot_pair);
  STRATA_CHECK_LAUNCH();
  if (nblocks > 0) {
    hipLaunchKernelGGL(route_place, dim3(nblocks), dim3(kBlock), 4 * lds_e, s, idx, (int)pairs, (int)k, (int)experts,
                       (int)tile, blk, first_tile, token, where, slot_pair);
    STRATA_CHECK_LAUNCH();
  }
  return STRATA_OK;
}

}  // extern "C"

extern "C" int strata_route_tiles_noalloc(const uint32_t* idx, int64_t pairs, int64_t k, int64_t experts, int64_t tile,
                                          uint32_t* tile_expert, uint32_t* token, uint32_t* where,
                                          uint32_t* slot_pair, void* stream) {
  if (pairs < 0 || k < 1 || experts < 1 || tile < 1 || tile > 1024) return STRATA_ERR_ARG;
  if (pairs > kScratchPairs || experts > kScratchExperts) return STRATA_ERR_SHAPE;
  if (strata_route_tiles_workspace(pairs, experts) > kScratchWords * (int64_t)sizeof(uint32_t)) return STRATA_ERR_SHAPE;
  void* ws = device_scratch();
  if (ws == nullptr) return STRATA_ERR_LAUNCH;
  return strata_route_tiles(idx, pairs, k, experts, tile, tile_expert, token, where, slot_pair, ws, stream);
}
