// The dense one-token matvec of a long Q6_K matrix (an lm_head: 151936 rows of 4096 inputs, 510 MB; q, k and v
// fused: 12288 rows) with each row staged in LDS by contiguous 16-byte direct loads (strata_mlx/dense.py:109-167, ScaledLinear at one token,
// whose weights are the file's Q6_K blocks, strata_mlx/gguf.py:150-165).
//
// Read straight into registers (direct_decode_kernel), a lane's run pair takes seven field loads (d, two scales,
// two 16-byte pieces of the low bits and two of the high bits), and each of them touches all 27 cache lines of
// the row's 3360 bytes, since the row's 64 lanes read at 16 blocks of 210 bytes. On the lm_head that kept the
// texture units busy for most of the launch (TA 76 %, TD 86 %, 53 TD cycles a load instruction), with HBM at
// 0.52 of its peak. Here a row is four wave instructions of 1 KB each (global_load_lds_dwordx4: lane l's 16
// bytes land at M0 + 16 l), and the lanes read their fields from LDS: the lm_head 122-125 -> 100-101 us, q/k/v
// 12.7-13.0 -> 11.9-12.2 us. Two or four slabs a wave in place of three measured the same or slower.
//
// Each wave streams its own rows (w, w + waves, ...) through SLABS slabs of its own: the rows of the next
// SLABS - 1 slabs are in flight while one is decoded, so no workgroup barrier is needed anywhere, and one wait
// (vmcnt) a row. The LDS reads are naturally aligned dwords put together by v_alignbyte: a 210-byte block starts
// at an even byte, and misaligned 8- or 16-byte LDS reads run many times slower. A layer this kernel takes has
// its listed rows (row_ids, strata_mlx/rows.py:30-42) taken here too, so that a listed row has the bits of the
// same row of the full product (the direct kernel's bits differ in the last place for about 1 % of the rows).
#pragma once

namespace strata_mv {

constexpr int kStreamWaves = 4;          // waves a workgroup
constexpr int kStreamSlab = 4096;        // LDS bytes a slab: a row of up to 4096 bytes (four 1 KB loads)
constexpr int kStreamLoads = kStreamSlab / 1024;

template <int SLABS>
constexpr int stream_lds() {
  return kStreamWaves * SLABS * kStreamSlab;
}

// lane l's 16 bytes at base + voff into LDS at lds + 16 l (the wave's LDS address in M0); NT: with the
// non-temporal (streaming) cache policy, for rows read once that the caches need not keep
template <bool NT>
__device__ __forceinline__ void dma_x4(const uint8_t* base, uint32_t voff, uint8_t* lds) {
  __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)(base + voff),
                                   (__attribute__((address_space(3))) void*)lds, 16, 0, NT ? 2 : 0);
}

// N 32-bit words from byte offset off of LDS (off even): N + 1 aligned dwords, shifted by off % 4 bytes.
template <int N>
__device__ __forceinline__ void lds_words(const uint8_t* base, uint32_t off, uint32_t (&w)[N]) {
  const uint32_t* p = reinterpret_cast<const uint32_t*>(base + (off & ~3u));
  const uint32_t sh = off & 3u;
  uint32_t d[N + 1];
#pragma unroll
  for (int k = 0; k <= N; ++k) d[k] = p[k];
#pragma unroll
  for (int k = 0; k < N; ++k) w[k] = __builtin_amdgcn_alignbyte(d[k + 1], d[k], sh);
}

// Lane j's run pair of a Q6_K row staged at `row` in LDS (offsets of lane_offsets: ql @qs, qh @a, the scales
// @b and b + 4, d @d).
__device__ __forceinline__ void stream_fields(const uint8_t* row, const LaneOffsets<K_Q6_K>& o, RunPair<K_Q6_K>& f) {
  uint32_t ql[8], qh[8], sc[2], d[1];
  lds_words<8>(row, o.qs, ql);
  lds_words<8>(row, o.a, qh);
  lds_words<2>(row, o.b, sc);
  lds_words<1>(row, o.d, d);
  f.ql[0] = u32x4{ql[0], ql[1], ql[2], ql[3]};
  f.ql[1] = u32x4{ql[4], ql[5], ql[6], ql[7]};
  f.qh[0] = u32x4{qh[0], qh[1], qh[2], qh[3]};
  f.qh[1] = u32x4{qh[4], qh[5], qh[6], qh[7]};
  f.sc[0] = (uint16_t)(sc[0] & 0xFFFFu);
  f.sc[1] = (uint16_t)(sc[1] & 0xFFFFu);
  f.d = (uint16_t)(d[0] & 0xFFFFu);
}

struct StreamParams {
  const uint8_t* blocks;  // src_rows x row_bytes
  const u32x4* x;         // the token: cols float16
  f16* out;               // rows float16
  const uint32_t* ids;    // the rows to compute (an id past the matrix reads row 0 and writes NaN), or null: all
  int rows, src_rows, row_bytes;
};

template <int KIND, int SLABS, bool NT>
__global__ __launch_bounds__(64 * kStreamWaves) void stream_rows_kernel(StreamParams p) {
  static_assert(KIND == K_Q6_K, "Q6_K rows of 4096 inputs");
  static_assert(SLABS >= 2 && SLABS <= 4, "the waits below count 4 loads a slab for up to three slabs in flight");
  __shared__ __attribute__((aligned(16))) uint8_t lds[stream_lds<SLABS>()];
  __shared__ DirectTables<KIND> tab;  // the linear types decode without it
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int waves = gridDim.x * kStreamWaves;
  const int w0 = blockIdx.x * kStreamWaves + wave;
  uint8_t* const slabs = lds + wave * SLABS * kStreamSlab;

  // the lane's 64 activations (runs run_of(lane, 0) and (lane, 1)) and their sums, before any row is asked for
  uint32_t x[32];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int r = run_of<KIND>(lane, h);
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const u32x4 c = p.x[4 * r + v];
#pragma unroll
      for (int i = 0; i < 4; ++i) x[16 * h + 4 * v + i] = c[i];
    }
  }
  float xsum[2 * kXSums<KIND> + 1];
  x_sums<KIND>(x, xsum);
  x_sums<KIND>(x + 16, xsum + kXSums<KIND>);
  // the sums are taken here, so the token's loads are waited for before any row's (not behind them)
  asm volatile("" : "+v"(xsum[0]), "+v"(xsum[1]), "+v"(xsum[2]), "+v"(xsum[3])::"memory");

  // row r's bytes into slab s: four 1 KB pieces; the lanes past the row read its last 16 bytes again (into the
  // slab's spare bytes)
  const uint32_t last = (uint32_t)p.row_bytes - 16u;
  auto source = [&](int r) {  // the matrix row of output row r (r past the last: the last again)
    const int q = min(r, p.rows - 1);
    if (p.ids == nullptr) return q;
    const uint32_t id = p.ids[q];
    return id < (uint32_t)p.src_rows ? (int)id : 0;
  };
  auto stage = [&](int r, int s) {
    const uint8_t* row = p.blocks + (int64_t)source(r) * p.row_bytes;
#pragma unroll
    for (int k = 0; k < kStreamLoads; ++k)
      dma_x4<NT>(row, min(1024u * k + 16u * lane, last), slabs + s * kStreamSlab + 1024 * k);
  };
#pragma unroll
  for (int s = 0; s < SLABS - 1; ++s) stage(w0 + s * waves, s);

  const LaneOffsets<KIND> o = lane_offsets<KIND>(lane);
  for (int i = 0;; ++i) {
    const int r = w0 + i * waves;
    if (r >= p.rows) break;
    const int s = i % SLABS;
    // the row SLABS - 1 rows on goes out, then this row's loads are waited for (those after it may be in flight)
    stage(r + (SLABS - 1) * waves, (i + SLABS - 1) % SLABS);
    if constexpr (SLABS == 2)
      asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
    else if constexpr (SLABS == 3)
      asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
    else
      asm volatile("s_waitcnt vmcnt(12)" ::: "memory");
    RunPair<KIND> f;
    stream_fields(slabs + s * kStreamSlab, o, f);
    float acc = 0.0f;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      uint32_t w[16];
      const RunScale rs = decode_run<KIND>(f, h, lane, w, tab);
      acc += apply_run<KIND>(rs, w, x + 16 * h, xsum + kXSums<KIND> * h);
    }
    float v[1] = {acc};
    const float total = reduce_steps<64, 1, true>(v, lane);
    const bool past = p.ids != nullptr && p.ids[r] >= (uint32_t)p.src_rows;
    if (lane == 0) p.out[r] = from_f32<f16>(past ? __builtin_nanf("") : total);
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the rows asked for past the last are in before the wave ends
}

// Whether stream_rows_kernel takes a dense call: one float16 token against a Q6_K matrix of 4096 inputs and at
// least 8192 rows (q/k/v fused, an lm_head), all its rows or listed ones, one stack, rows at 16-byte boundaries. The choice
// rests on the matrix, not on how many rows are listed, so a listed row and the full product take one kernel.
template <int KIND>
bool stream_takes(const MatvecParams& p, int grid_y) {
  return KIND == K_Q6_K && p.mode == MODE_DENSE && p.tokens == 1 && p.cols == 4096 && p.row_bytes == 3360 &&
         p.src_rows >= 8192 && grid_y == 1 && ((uintptr_t)p.blocks[0] & 15) == 0 && ((uintptr_t)p.x & 15) == 0;
}

constexpr int kStreamSlabs = 3;
constexpr int kStreamPastCaches = 65536;  // rows from which the rows' loads take the non-temporal policy

template <int KIND>
int launch_stream(const MatvecParams& mp, hipStream_t s) {
  if constexpr (KIND != K_Q6_K) {
    (void)mp;
    (void)s;
    return STRATA_ERR_KIND;
  } else {
    StreamParams p;
    p.blocks = mp.blocks[0];
    p.x = reinterpret_cast<const u32x4*>(mp.x);
    p.out = reinterpret_cast<f16*>(mp.out[0]);
    p.ids = mp.row_ids;
    p.rows = mp.rows;
    p.src_rows = mp.src_rows;
    p.row_bytes = mp.row_bytes;
    // workgroups a CU as the LDS allows, one round of them
    const int per_cu = max(1, (160 * 1024) / (stream_lds<kStreamSlabs>() + 1024));
    const int groups = min(device_cus() * per_cu, (p.rows + kStreamWaves - 1) / kStreamWaves);
    // a matrix of 65536 rows or more (220 MB or more, an lm_head) streamed past the caches: lm_head 151936 x 4096
    // 94.9-95.3 -> 85.8-86.3 us; q/k/v (12288 rows) kept the usual policy, 2-3 % faster with it
    if (p.src_rows >= kStreamPastCaches)
      hipLaunchKernelGGL((stream_rows_kernel<KIND, kStreamSlabs, true>), dim3((unsigned)groups),
                         dim3(64 * kStreamWaves), 0, s, p);
    else
      hipLaunchKernelGGL((stream_rows_kernel<KIND, kStreamSlabs, false>), dim3((unsigned)groups),
                         dim3(64 * kStreamWaves), 0, s, p);
    STRATA_CHECK_LAUNCH();
    return STRATA_OK;
  }
}

}  // namespace strata_mv
