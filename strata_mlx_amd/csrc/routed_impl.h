// Routed gate and up with the SwiGLU for one token, on IQ3_S rows of 4096 inputs: the decode matvec of a
// mixture-of-experts layer at batch one (strata_mlx/blocks.py:958-975 with the SwiGLU of its down call,
// :222-236), as one persistent launch.
//
// What a launch of direct_decode_kernel spends at this shape is mostly fixed cost: a chain of dependent loads
// before the first row byte is asked for (the parameters, the pair's expert, the mode's branches), a prologue and
// an epilogue for every four row steps, and 1.5 rounds of single-shot waves. Here one workgroup of sixteen waves
// sits on each CU for the whole launch, and a wave takes UPW units (a unit: row r of the gate matrix and row r of
// the up matrix of one pair), all known when it starts: their experts are read at once, the rows of up to three
// units are in flight together (a fourth goes out once the first is decoded), and the units' sums are written at
// the end by one lane each (one SwiGLU evaluation a wave, not one a unit).
//
// Order of the loads. The codebook and the token are asked for first and the workgroup barrier waits for them
// alone; the rows go out after it. A CU's loads return in the order they were asked for, so rows asked for
// before the barrier put every wave's codebook load behind the other waves' rows: the barrier then passed at
// 3.4-9 us into the launch instead of about 1 us (per-wave timestamps), and nothing was decoded until then.
// For the same reason nothing of the decode may be moved above the barrier (opaque(): the compiler would
// otherwise compute the codebook addresses there and wait for the rows at the barrier).
//
// The codebook sits in LDS with its signs folded in: entry s << 9 | g is grid entry g (nine index bits) with
// sign bit b of s flipping weight b, four float16 integers, 8192 entries of 8 bytes. A group of four weights is
// then one LDS read, its address one shift of a 16-bit word whose low byte is the index byte and whose high byte
// is the ninth index bit and the four sign bits, put together by v_perm from the fields as loaded. (With a
// separate 16-entry sign table, a group was two reads, two address shifts and two XORs.) The table and the token
// take 72 KB of LDS; at more than 64 VGPRs a CU holds one such workgroup.
//
// Lane j of a wave holds run pair j of a row (64 weights, the same 128 bytes of the token for every unit); the
// gate row's partial sums and the up row's meet in one exchange of halves and then within the halves.
#pragma once
// Included by direct_impl.h ahead of the dispatch (it uses that file's fields, offsets and reductions).

namespace strata_mv {

constexpr int kGluThreads = 1024;  // sixteen waves a workgroup, one workgroup a CU
constexpr int kGluWaves = kGluThreads / 64;
constexpr int kGluGroupsPerCU = 1;
constexpr int kGluMaxUnits = 4;     // units a wave (straight-line code); more units: more waves
constexpr int kGluEntries = 8192;   // 512 grid entries x 16 sign nibbles

struct GluParams {
  const uint8_t* gate;
  const uint8_t* up;
  const uint32_t* idx;  // expert of each pair
  const u32x4* x;       // the token: 4096 float16 as 512 pieces of 16 bytes
  f16* out_gate;        // gate . x (may be null)
  f16* out_up;          // up . x (may be null)
  f16* h;               // silu(gate . x) * (up . x)
  int64_t mat_bytes;
  uint32_t experts;
  int rows, row_bytes, pairs, units, waves;
  int wave_pairs, wave_rows;  // waves / rows and waves % rows: from a wave's unit to its next
};

// Lane j's offsets within a row, without each field's constant offset in its block (that goes to the row's
// address, which the whole wave shares): the loads then take a scalar base and a 32-bit lane offset.
struct GluOffsets {
  uint32_t d, qs, qh, sg, sc;
};
__device__ __forceinline__ GluOffsets glu_offsets(int j) {
  const uint32_t b = (uint32_t)(j >> 2) * 110, jj = (uint32_t)j & 3;
  return GluOffsets{b, b + 16 * jj, b + 2 * jj, b + 8 * jj, b + 2 * (jj >> 1)};
}

// The fields of lane j's run pair in the row at `row` (IQ3_S: d @0, qs[64] @2, qh[8] @66, signs[32] @74,
// scales[4] @106 of each 110-byte block).
__device__ __forceinline__ void glu_load(const uint8_t* row, const GluOffsets& o, RunPair<K_IQ3_S>& f) {
  f.d = load_at<uint16_t>(row, o.d);
  f.qs = load_at<u32x4>(row + 2, o.qs);
  f.qh = load_at<uint16_t>(row + 66, o.qh);
  f.sg = load_at<u32x2>(row + 74, o.sg);
  f.sc = load_at<uint16_t>(row + 106, o.sc);
}

// Run h (0, 1) of the pair: its 32 weights from the signed codebook, times 32 activations (16 packed pairs).
// Group l's word: the index byte qs[l] low, the ninth bit and the sign nibble of group l high. The ninth bits
// of the even groups (bits 0, 2, 4, 6 of the run's qh byte) go to bit 0 of bytes 0..3 by one multiply (the
// products' other bits never reach bits 0, 8, 16, 24), the sign nibbles of the even groups are the low nibbles of
// the run's four sign bytes; the odd groups take bits 1, 3, 5, 7 and the high nibbles.
__device__ __forceinline__ float iq3s_run_signed(const RunPair<K_IQ3_S>& f, int h, const uint32_t* x,
                                                 const u32x2* tab) {
  const uint32_t q0 = f.qs[2 * h], q1 = f.qs[2 * h + 1];
  const uint32_t hb = (uint32_t)f.qh >> (8 * h);
  const uint32_t sg = f.sg[h];
  const uint32_t he = (((hb & 0x55u) * 0x41041u) & 0x01010101u) | ((sg & 0x0F0F0F0Fu) << 1);
  const uint32_t ho = ((((hb >> 1) & 0x55u) * 0x41041u) & 0x01010101u) | ((sg >> 3) & 0x1E1E1E1Eu);
  const uint32_t w02 = __builtin_amdgcn_perm(he, q0, 0x05020400u), w13 = __builtin_amdgcn_perm(ho, q0, 0x05030401u);
  const uint32_t w46 = __builtin_amdgcn_perm(he, q1, 0x07020600u), w57 = __builtin_amdgcn_perm(ho, q1, 0x07030601u);
  const uint32_t three = 3;
  const uint32_t a[8] = {word_shl<0>(w02, three), word_shl<0>(w13, three), word_shl<1>(w02, three),
                         word_shl<1>(w13, three), word_shl<0>(w46, three), word_shl<0>(w57, three),
                         word_shl<1>(w46, three), word_shl<1>(w57, three)};
  uint32_t w[16];
#pragma unroll
  for (int l = 0; l < 8; ++l) {
    const u32x2 v = lds_entry(tab, a[l]);
    w[2 * l] = v[0];
    w[2 * l + 1] = v[1];
  }
  return dot16x2(w, x + 16 * h);
}

// Lane j's share of a row: its two runs, each times its scale d (1 + 2 s).
__device__ __forceinline__ float iq3s_pair_signed(const RunPair<K_IQ3_S>& f, int j, const uint32_t* x,
                                                  const u32x2* tab) {
  const float d = half_bits(f.d);
  const uint32_t sc = (uint32_t)f.sc >> (8 * (j & 1));
  const float s0 = d * (float)(1 + 2 * (sc & 15u)), s1 = d * (float)(1 + 2 * ((sc >> 4) & 15u));
  return s0 * iq3s_run_signed(f, 0, x, tab) + s1 * iq3s_run_signed(f, 1, x, tab);
}

// The unit's two rows decoded and multiplied, and their sums met over the wave: the gate row's total and the up
// row's, the same in every lane (read once into scalars).
template <int KIND>
__device__ __forceinline__ void glu_unit(RunPair<KIND> (&f)[2], int lane, const uint32_t* x, const u32x2* tab,
                                         float& gate, float& up) {
  opaque(f[0]);  // nothing of the decode is done before the workgroup barrier (it would wait for these rows there)
  opaque(f[1]);
  float g = iq3s_pair_signed(f[0], lane, x, tab);
  float u = iq3s_pair_signed(f[1], lane, x, tab);
  // lanes 0-31 the gate row's partial sums two at a time, lanes 32-63 the up row's; then within the halves
  float v = sum_swapped(g, u, 32);
  v = sum_swapped(v, v, 16);
  v += lanes_apart(v, 8);
  v += lanes_apart(v, 4);
  v += lanes_apart(v, 2);
  v += lanes_apart(v, 1);
  gate = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__float_as_int(v), 0));
  up = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__float_as_int(v), 32));
}

// The token in LDS: piece c (16 bytes) of lane j = c / 8 at slot 8 j + (c % 8 ^ j % 8), so that the eight lanes
// of one LDS cycle of a 16-byte read fall on distinct banks.
__device__ __forceinline__ int glu_x_slot(int j, int i) { return 8 * j + (i ^ (j & 7)); }

template <int KIND, int UPW>
__global__ __launch_bounds__(kGluThreads, 4) void routed_glu_kernel(GluParams p) {
  static_assert(KIND == K_IQ3_S, "the signed codebook is IQ3_S's");
  constexpr int kBuffers = UPW < 3 ? UPW : 3;  // units whose rows are in registers at once
  __shared__ u32x2 tab[kGluEntries];
  __shared__ u32x4 xs[512];
  const int tid = threadIdx.x, lane = tid & 63;
  const int gw = blockIdx.x * kGluWaves + __builtin_amdgcn_readfirstlane(tid >> 6);

  // what the workgroup shares, asked for first: the codebook entry this thread expands and a piece of the token
  const uint64_t entry = kIq3sHalfGrid.v[tid & 511];
  const u32x4 xpiece = p.x[tid & 511];
  // the wave's units and their experts
  int pair[UPW], row[UPW];
  bool live[UPW];
  {
    int pr = gw / p.rows, r = gw - pr * p.rows;
#pragma unroll
    for (int k = 0; k < UPW; ++k) {
      live[k] = pr < p.pairs;
      pair[k] = live[k] ? pr : p.pairs - 1;  // past the last unit: the last unit's rows again, nothing written
      row[k] = live[k] ? r : p.rows - 1;
      r += p.wave_rows;
      pr += p.wave_pairs;
      if (r >= p.rows) {
        r -= p.rows;
        ++pr;
      }
    }
  }
  uint32_t expert[UPW];
  bool bad[UPW];
#pragma unroll
  for (int k = 0; k < UPW; ++k) {
    const uint32_t e = p.idx[pair[k]];
    bad[k] = e >= p.experts;
    expert[k] = bad[k] ? 0u : e;  // a pair naming no expert reads expert 0's rows and writes NaN
  }
  const GluOffsets lo = glu_offsets(lane);
  auto issue = [&](int k, RunPair<KIND>(&f)[2]) {
    const int64_t off = (int64_t)expert[k] * p.mat_bytes + (int64_t)row[k] * p.row_bytes;
    glu_load(p.gate + off, lo, f[0]);
    glu_load(p.up + off, lo, f[1]);
    asm volatile("" ::: "memory");  // the units' loads go out in unit order
  };

  // the signed codebook: this thread's grid entry under eight of the 16 sign nibbles; the token's pieces
  {
    const uint32_t lo32 = (uint32_t)entry, hi32 = (uint32_t)(entry >> 32);
    const int half = tid >> 9;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int s = 8 * half + i;
      const uint32_t m0 = ((i & 1) ? 0x8000u : 0u) | ((i & 2) ? 0x80000000u : 0u);
      const uint32_t m1 = ((i & 4) ? 0x8000u : 0u) | (half ? 0x80000000u : 0u);
      tab[s * 512 + (tid & 511)] = u32x2{lo32 ^ m0, hi32 ^ m1};
    }
    xs[glu_x_slot((tid & 511) >> 3, tid & 7)] = xpiece;  // two threads a piece: the same bytes
  }
  __syncthreads();
  uint32_t x[32];
#pragma unroll
  for (int v = 0; v < 8; ++v) {
    const u32x4 c = xs[glu_x_slot(lane, v)];
#pragma unroll
    for (int i = 0; i < 4; ++i) x[4 * v + i] = c[i];
  }
  RunPair<KIND> f[kBuffers][2];
#pragma unroll
  for (int k = 0; k < kBuffers; ++k) issue(k, f[k]);

  float gate[UPW], up[UPW];
#pragma unroll
  for (int k = 0; k < UPW; ++k) {
    glu_unit<KIND>(f[k % kBuffers], lane, x, tab, gate[k], up[k]);
    if (k + kBuffers < UPW) issue(k + kBuffers, f[k % kBuffers]);
  }

  // lane k writes unit k: gate, up and silu(gate) * up as mlx-lm rounds it
  float gv = gate[0], uv = up[0];
#pragma unroll
  for (int k = 1; k < UPW; ++k) {
    gv = lane == k ? gate[k] : gv;
    uv = lane == k ? up[k] : uv;
  }
  int my = 0;
#pragma unroll
  for (int k = 1; k < UPW; ++k) my = lane == k ? k : my;
  bool w_live = false, w_bad = false;
  int w_pair = 0, w_row = 0;
#pragma unroll
  for (int k = 0; k < UPW; ++k) {
    if (my == k) {
      w_live = live[k];
      w_bad = bad[k];
      w_pair = pair[k];
      w_row = row[k];
    }
  }
  if (lane < UPW && w_live) {
    const int64_t o = (int64_t)w_pair * p.rows + w_row;
    f16 gq = from_f32<f16>(gv), uq = from_f32<f16>(uv), hq;
    if (w_bad) {
      gq = uq = hq = (f16)__builtin_nanf("");
    } else {
      hq = from_f32<f16>(swiglu_rounded<f16>(gq, uq));
    }
    if (p.out_gate != nullptr) p.out_gate[o] = gq;
    if (p.out_up != nullptr) p.out_up[o] = uq;
    p.h[o] = hq;
  }
}

// Down (and any one-matrix routed product) on IQ3_S rows of 1536 or 2560 inputs: 8 lanes take a row, lane m its
// run pairs m, m + 8, ... (S of them), so a wave holds 8 rows (a unit). A workgroup (one a CU) takes consecutive
// units of one pair, whose token sits in LDS beside the signed codebook; the rows go out after the barrier, as
// in routed_glu_kernel, and a row's sum meets over its 8 lanes by three DPP steps.
struct DownParams {
  const uint8_t* blocks;
  const uint32_t* idx;
  const f16* x;  // pairs / share tokens of 512 S float16
  f16* out;
  int64_t mat_bytes;
  uint32_t experts;
  int rows, row_bytes, pairs, share;
  int groups_per_pair;  // workgroups a pair
};

template <int S, int UPW>
__global__ __launch_bounds__(kGluThreads, 4) void routed_down_kernel(DownParams p) {
  constexpr int kPairs = 8 * S;        // run pairs of a row
  constexpr int kPieces = 8 * kPairs;  // 16-byte pieces of a token
  __shared__ u32x2 tab[kGluEntries];
  __shared__ u32x4 xs[kPieces];
  const int tid = threadIdx.x, lane = tid & 63, m = lane & 7, sub = lane >> 3;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int pair = blockIdx.x / p.groups_per_pair, chunk = blockIdx.x - pair * p.groups_per_pair;

  // the codebook entry this thread expands and a piece of the pair's token, asked for first
  const uint64_t entry = kIq3sHalfGrid.v[tid & 511];
  const u32x4 xpiece = reinterpret_cast<const u32x4*>(p.x + (int64_t)(pair / p.share) * (8 * kPieces))[tid % kPieces];
  const uint32_t e = p.idx[pair];
  const bool bad = e >= p.experts;
  const uint8_t* mat = p.blocks + (int64_t)(bad ? 0u : e) * p.mat_bytes;
  int r0[UPW];
#pragma unroll
  for (int k = 0; k < UPW; ++k) r0[k] = ((chunk * kGluWaves + wave) * UPW + k) * 8;  // the unit's first row
  {
    const uint32_t lo32 = (uint32_t)entry, hi32 = (uint32_t)(entry >> 32);
    const int half = tid >> 9;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int s = 8 * half + i;
      const uint32_t m0 = ((i & 1) ? 0x8000u : 0u) | ((i & 2) ? 0x80000000u : 0u);
      const uint32_t m1 = ((i & 4) ? 0x8000u : 0u) | (half ? 0x80000000u : 0u);
      tab[s * 512 + (tid & 511)] = u32x2{lo32 ^ m0, hi32 ^ m1};
    }
    const int c = tid % kPieces;  // threads past the token's pieces write the same bytes again
    xs[glu_x_slot(c >> 3, c & 7)] = xpiece;
  }
  __syncthreads();

  RunPair<K_IQ3_S> f[UPW][S];
#pragma unroll
  for (int k = 0; k < UPW; ++k) {
    const int rl = min(r0[k] + sub, p.rows - 1);  // rows past the matrix read its last row, and write nothing
    const uint8_t* row = mat + (int64_t)rl * p.row_bytes;
#pragma unroll
    for (int st = 0; st < S; ++st) glu_load(row, glu_offsets(8 * st + m), f[k][st]);
    asm volatile("" ::: "memory");
  }
#pragma unroll
  for (int k = 0; k < UPW; ++k) {
    float acc = 0.0f;
#pragma unroll
    for (int st = 0; st < S; ++st) {
      opaque(f[k][st]);
      const int j = 8 * st + m;
      uint32_t x[32];
#pragma unroll
      for (int v = 0; v < 8; ++v) {
        const u32x4 c = xs[glu_x_slot(j, v)];
#pragma unroll
        for (int i = 0; i < 4; ++i) x[4 * v + i] = c[i];
      }
      acc += iq3s_pair_signed(f[k][st], j, x, tab);
    }
    acc += lanes_apart(acc, 1);
    acc += lanes_apart(acc, 2);
    acc += lanes_apart(acc, 4);
    const int r = r0[k] + sub;
    if (m == 0 && r < p.rows) p.out[(int64_t)pair * p.rows + r] = bad ? (f16)__builtin_nanf("") : from_f32<f16>(acc);
  }
}

// Whether routed_down_kernel takes a routed one-matrix call: IQ3_S rows of 1536 or 2560 inputs, float16 in and
// out (the caller has checked the dtypes).
template <int KIND>
bool routed_down_takes(const MatvecParams& p) {
  return KIND == K_IQ3_S && p.mode == MODE_EXPERT && (p.cols == 1536 || p.cols == 2560) &&
         p.glu_out == nullptr && p.experts <= INT32_MAX && p.pairs <= 65535;
}

template <int S, int UPW>
int launch_down_su(DownParams& p, int units_per_pair, hipStream_t s) {
  const int per_group = kGluWaves * UPW;
  p.groups_per_pair = (units_per_pair + per_group - 1) / per_group;
  const int64_t groups = (int64_t)p.groups_per_pair * p.pairs;
  if (groups > INT32_MAX) return STRATA_ERR_SHAPE;
  hipLaunchKernelGGL((routed_down_kernel<S, UPW>), dim3((unsigned)groups), dim3(kGluThreads), 0, s, p);
  STRATA_CHECK_LAUNCH();
  return STRATA_OK;
}

template <int KIND>
int launch_routed_down(const MatvecParams& mp, hipStream_t s) {
  if constexpr (KIND != K_IQ3_S) {
    return STRATA_ERR_SHAPE;
  } else {
    DownParams p = {};
    p.blocks = mp.blocks[0];
    p.idx = mp.idx;
    p.x = reinterpret_cast<const f16*>(mp.x);
    p.out = reinterpret_cast<f16*>(mp.out[0]);
    p.mat_bytes = mp.mat_bytes;
    p.experts = (uint32_t)mp.experts;
    p.rows = mp.rows;
    p.row_bytes = mp.row_bytes;
    p.pairs = mp.pairs;
    p.share = mp.share;
    const int units_per_pair = (mp.rows + 7) / 8;
    const int64_t units = (int64_t)units_per_pair * mp.pairs;
    const int64_t capacity = (int64_t)device_cus() * kGluGroupsPerCU * kGluWaves;
    const bool two = units > capacity;  // more units than one round of waves: two a wave
    if (mp.cols == 1536) return two ? launch_down_su<3, 2>(p, units_per_pair, s) : launch_down_su<3, 1>(p, units_per_pair, s);
    return two ? launch_down_su<5, 2>(p, units_per_pair, s) : launch_down_su<5, 1>(p, units_per_pair, s);
  }
}

// Whether routed_glu_kernel takes a paired gate/up call: IQ3_S rows of 4096 inputs, one token for every pair,
// float16 in and out (the caller has checked the dtypes).
template <int KIND>
bool routed_glu_takes(const MatvecParams& p) {
  return KIND == K_IQ3_S && p.mode == MODE_EXPERT && p.cols == 4096 && p.share == p.pairs && p.glu_out != nullptr &&
         p.experts <= INT32_MAX && (int64_t)p.pairs * p.rows <= INT32_MAX / 2;
}

template <int KIND>
int launch_routed_glu(const MatvecParams& mp, hipStream_t s) {
  if constexpr (KIND != K_IQ3_S) {
    return STRATA_ERR_SHAPE;
  } else {
    GluParams p = {};
    p.gate = mp.blocks[0];
    p.up = mp.blocks[1];
    p.idx = mp.idx;
    p.x = reinterpret_cast<const u32x4*>(mp.x);
    p.out_gate = reinterpret_cast<f16*>(mp.out[0]);
    p.out_up = reinterpret_cast<f16*>(mp.out[1]);
    p.h = reinterpret_cast<f16*>(mp.glu_out);
    p.mat_bytes = mp.mat_bytes;
    p.experts = (uint32_t)mp.experts;
    p.rows = mp.rows;
    p.row_bytes = mp.row_bytes;
    p.pairs = mp.pairs;
    p.units = mp.pairs * mp.rows;
    const int capacity = device_cus() * kGluGroupsPerCU * kGluWaves;
    int upw = (p.units + capacity - 1) / capacity;
    upw = upw < 1 ? 1 : (upw > kGluMaxUnits ? kGluMaxUnits : upw);
    const int64_t waves = ((int64_t)(p.units + upw - 1) / upw + kGluWaves - 1) / kGluWaves * kGluWaves;
    if (waves / kGluWaves > INT32_MAX) return STRATA_ERR_SHAPE;
    p.waves = (int)waves;
    p.wave_pairs = p.waves / p.rows;
    p.wave_rows = p.waves % p.rows;
    const dim3 grid((unsigned)(waves / kGluWaves));
    switch (upw) {
      case 1: hipLaunchKernelGGL((routed_glu_kernel<KIND, 1>), grid, dim3(kGluThreads), 0, s, p); break;
      case 2: hipLaunchKernelGGL((routed_glu_kernel<KIND, 2>), grid, dim3(kGluThreads), 0, s, p); break;
      case 3: hipLaunchKernelGGL((routed_glu_kernel<KIND, 3>), grid, dim3(kGluThreads), 0, s, p); break;
      default: hipLaunchKernelGGL((routed_glu_kernel<KIND, 4>), grid, dim3(kGluThreads), 0, s, p); break;
    }
    STRATA_CHECK_LAUNCH();
    return STRATA_OK;
  }
}

}  // namespace strata_mv
