// Grouped expert FFN for decode-sized groups (a few tokens per expert).
//
// Replaces the same per-expert GEMMs as the tiled kernel
// (reframework/moe/fused.py:76-83) when each expert sees <= ~32 rows. Then the
// layer is a weight stream: every routed expert's 3*H*I weights are read once
// and meet only a handful of tokens, so the kernel is built for HBM bandwidth.
//
// Each wave owns 16 weight rows (gate_up: 16 gate rows + the 16 matching up
// rows) of one expert and one 16-token tile, and multiplies with
// v_mfma_f32_16x16x32 (weights on the M side, tokens on the N side).
//
// Weight loads are shaped for DRAM, not for the MFMA operand: one load
// instruction reads 4 rows x 256 contiguous bytes (16 lanes per row), so a
// 128-element k step of 16 rows is 4 instructions. The wave stages them in its
// own slice of LDS, each row's 16-byte chunks XOR-permuted by the row index, and
// reads them back in the MFMA layout (lane l: row l%16, chunk 4s + l/16), which
// the permutation makes bank-conflict free. The 16 lanes of one row fetch the
// row's chunks in permuted order, so each row still reads one contiguous
// 256-byte run. Loading the operand directly in MFMA layout would split every
// instruction into 16 separate 64-byte pieces, which measured ~5 TB/s instead of
// ~7 TB/s on MI355X.
//
// Steps are prefetched D deep in registers, LDS slices are double-buffered, and
// each wave starts its K walk at a rotated step so that concurrent waves hit
// different HBM channels. No workgroup barrier is needed: every wave only
// reads what it wrote. gate_up fuses the gated activation; down writes fp32
// partials per K-split, which the combine kernel sums, so the short down
// projection of a decode step still spreads over every CU.
#include <climits>

#include "common.h"

namespace moe355 {
namespace {

constexpr int kThreads = 256;
constexpr int kWavesPerBlock = kThreads / kWave;
constexpr int kRows = 16;
constexpr int kKS = 128;                 // k elements per step
constexpr int kRowStepBytes = kKS * 2;   // 256 bytes of one row per step
constexpr int kOperandBytes = kRows * kRowStepBytes;  // 4 KB

template <typename T>
struct Mfma16;

template <>
struct Mfma16<bf16> {
  __device__ __forceinline__ static f32x4 mma(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
};

template <>
struct Mfma16<f16> {
  __device__ __forceinline__ static f32x4 mma(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
};

__device__ __forceinline__ u32x4 load16(const void* p) {
  return *reinterpret_cast<const u32x4*>(p);
}

__device__ __forceinline__ u32x4 load16_stream(const void* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}

// Grouping of <= 64 routed slots by one wave, the same stable counting sort
// as the permute kernels (experts ascending, slots ascending within an
// expert): lane s holds slot s. Each slot ORs its bit into its expert's 64-bit
// mask in LDS; an expert's row count is its mask's popcount and a slot's rank
// among its expert's slots the popcount of the mask bits below it, so no step
// depends on how many distinct experts there are. Lane l owns experts 4 l ..
// 4 l + 3 (E <= 256); one wave scan gives every expert's first row and first
// tile. Returns, for token tile ttile, its expert, first row and row end in
// meta[1..3] and the tile count in meta[0]; rowsrc[row] = source token of each
// permuted row. With write_global the wave also writes the permute's outputs
// (offsets, slot_to_row, row_src, tile_map with kRows-row tiles in expert
// order) for the later stages.
constexpr int kGroupExpertsPerLane = 4;
static_assert(kGroupExpertsPerLane * kWave >= kMaxExperts, "experts per lane");

__device__ void group_slots(const PermuteArgs& pa, int ttile, bool write_global, int* meta,
                            int* rowsrc, unsigned long long* emask, int* estart) {
  const int lane = threadIdx.x & (kWave - 1);
  constexpr int P = kGroupExpertsPerLane;
#pragma unroll
  for (int i = 0; i < P; ++i) emask[P * lane + i] = 0ull;
  const int e = lane < pa.R ? routed_expert(pa, lane) : -1;
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  if (e >= 0) atomicOr(&emask[e], 1ull << lane);
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  // this lane's experts: row counts and tile counts, then exclusive scans
  int cnt[P], nt[P], rows = 0, tiles = 0;
#pragma unroll
  for (int i = 0; i < P; ++i) {
    const int x = P * lane + i;
    cnt[i] = x < pa.E ? __popcll(emask[x]) : 0;
    nt[i] = (cnt[i] + kRows - 1) / kRows;
    rows += cnt[i];
    tiles += nt[i];
  }
  int rscan = rows, tscan = tiles;
#pragma unroll
  for (int o = 1; o < kWave; o <<= 1) {
    const int rv = __shfl_up(rscan, o, kWave), tv = __shfl_up(tscan, o, kWave);
    if (lane >= o) {
      rscan += rv;
      tscan += tv;
    }
  }
  const int total_rows = __shfl(rscan, kWave - 1, kWave);
  const int total_tiles = __shfl(tscan, kWave - 1, kWave);
  int rstart = rscan - rows, tstart = tscan - tiles;
  if (lane == 0) {
    meta[0] = total_tiles;
    meta[1] = -1;
    meta[2] = 0;
    meta[3] = 0;
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
  for (int i = 0; i < P; ++i) {
    const int x = P * lane + i;
    if (x < pa.E) {
      estart[x] = rstart;
      if (ttile >= tstart && ttile < tstart + nt[i]) {
        const int r0 = rstart + (ttile - tstart) * kRows;
        meta[1] = x;
        meta[2] = r0;
        meta[3] = min(r0 + kRows, rstart + cnt[i]);
      }
      if (write_global) {
        pa.offsets[x] = rstart;
        for (int j = 0; j < nt[i]; ++j) {
          pa.tile_map[2 + 2 * (tstart + j)] = x;
          pa.tile_map[3 + 2 * (tstart + j)] = rstart + j * kRows;
        }
      }
    }
    rstart += cnt[i];
    tstart += nt[i];
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  const unsigned long long lt_mask = (1ull << lane) - 1ull;
  const int row = e >= 0 ? estart[e] + __popcll(emask[e] & lt_mask) : -1;
  if (row >= 0) rowsrc[row] = lane / pa.K;
  if (!write_global) return;
  if (lane < pa.R) pa.slot_to_row[lane] = row;
  if (row >= 0) pa.row_src[row] = lane / pa.K;
  if (lane == 0) {
    pa.offsets[pa.E] = total_rows;
    pa.tile_map[0] = total_tiles;
    pa.tile_map[1] = kRows;
  }
}

template <typename T, bool kGateUp, bool kSelfPermute>
__global__ __launch_bounds__(kThreads) void ffn_skinny_kernel(const FfnArgs a) {
  constexpr int NOP = kGateUp ? 2 : 1;   // weight operands: gate (+ up)
  constexpr int D = kGateUp ? 2 : 4;     // steps in flight per wave
  constexpr int kSliceBytes = NOP * kOperandBytes;
  __shared__ __attribute__((aligned(16))) uint8_t lds[kWavesPerBlock][2][kSliceBytes];

  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
  const int group = blockIdx.x * kWavesPerBlock + wave;
  const int ttile = blockIdx.y, split = blockIdx.z;
  int e, row0, row_end;
  __shared__ int s_meta[4], s_rowsrc[kWave], s_estart[kGroupExpertsPerLane * kWave];
  __shared__ unsigned long long s_emask[kGroupExpertsPerLane * kWave];
  if (kSelfPermute) {
    // Every wave reaches the barrier before any returns.
    if (wave == 0)
      group_slots(a.perm, ttile, blockIdx.x == 0 && blockIdx.y == 0 && blockIdx.z == 0, s_meta,
                  s_rowsrc, s_emask, s_estart);
    __syncthreads();
    if (ttile >= s_meta[0] || group >= a.n_wtiles) return;
    e = s_meta[1];
    row0 = s_meta[2];
    row_end = s_meta[3];
  } else {
    if (ttile >= a.tile_map[0] || group >= a.n_wtiles) return;
    e = a.tile_map[2 + 2 * ttile];
    row0 = a.tile_map[3 + 2 * ttile];
    row_end = min(row0 + kRows, a.offsets[e + 1]);
  }

  const int ld = kGateUp ? a.H : a.I;
  const int kbeg = split * a.k_per_split;
  const int nsteps = a.k_per_split / kKS;

  // Operand o covers weight rows base(o) .. base(o)+15.
  const T* w = static_cast<const T*>(a.w[e]);
  const T* wop[NOP];
  wop[0] = w + static_cast<size_t>(group * kRows) * ld;
  if (kGateUp) wop[NOP - 1] = w + static_cast<size_t>(a.I + group * kRows) * ld;

  // Load j of a step: this lane reads row 4j + lane/16, logical chunk
  // (lane%16) ^ row, so the 16 lanes of a row cover its 256 bytes.
  uint32_t goff[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int r = 4 * j + (lane >> 4);
    goff[j] = static_cast<uint32_t>(r * ld + (((lane & 15) ^ r) * 8));
  }
  // MFMA sub-step s reads row lane%16, logical chunk 4s + lane/16.
  uint32_t roff[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    const int r = lane & 15, c = 4 * s + (lane >> 4);
    roff[s] = static_cast<uint32_t>(r * kRowStepBytes + ((c ^ r) << 4));
  }

  const int prow = row0 + (lane & 15);
  const bool valid = prow < row_end;
  const int xrow = !kGateUp     ? (valid ? prow : row0)
                   : kSelfPermute ? s_rowsrc[valid ? prow : row0]
                                  : a.row_src[valid ? prow : row0];
  const T* xp = static_cast<const T*>(a.x) + static_cast<size_t>(xrow) * ld + (lane >> 4) * 8;
  const u32x4 zero = {0, 0, 0, 0};

  // Rotated walk over the K steps of this split.
  const int s0 = nsteps > 0 ? (group * 7 + split * 3) % nsteps : 0;

  u32x4 wr[D][NOP][4], xr[D][4];
  auto issue = [&](int slot, int st) {
    int idx = s0 + st;
    if (idx >= nsteps) idx -= nsteps;
    const int k = kbeg + idx * kKS;
#pragma unroll
    for (int o = 0; o < NOP; ++o)
#pragma unroll
      for (int j = 0; j < 4; ++j) wr[slot][o][j] = load16_stream(wop[o] + k + goff[j]);
#pragma unroll
    for (int s = 0; s < 4; ++s) xr[slot][s] = valid ? load16(xp + k + s * 32) : zero;
  };

  f32x4 acc[NOP];
#pragma unroll
  for (int o = 0; o < NOP; ++o) acc[o] = f32x4{0.f, 0.f, 0.f, 0.f};

  auto consume = [&](int slot) {
    uint8_t* buf = lds[wave][slot & 1];
#pragma unroll
    for (int o = 0; o < NOP; ++o)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        *reinterpret_cast<u32x4*>(buf + o * kOperandBytes + (64 * j + lane) * 16) = wr[slot][o][j];
    // The wave reads back what it just wrote: order the LDS accesses.
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
      for (int o = 0; o < NOP; ++o) {
        const u32x4 fa = *reinterpret_cast<const u32x4*>(buf + o * kOperandBytes + roff[s]);
        acc[o] = Mfma16<T>::mma(fa, xr[slot][s], acc[o]);
      }
  };

#pragma unroll
  for (int d = 0; d < D; ++d)
    if (d < nsteps) issue(d, d);
  for (int st = 0; st < nsteps; st += D) {
#pragma unroll
    for (int d = 0; d < D; ++d) {
      if (st + d < nsteps) {
        consume(d);
        if (st + d + D < nsteps) issue(d, st + d + D);
      }
    }
  }

  // Lane (row, kq) holds features 4*kq + 0..3 of this 16-row group for token lane%16.
  if (!valid) return;
  const int col = group * kRows + 4 * (lane >> 4);
  if (kGateUp) {
    const f32x4 g = acc[0], u = acc[NOP - 1];
    T* inter = static_cast<T*>(a.out) + static_cast<size_t>(prow) * a.I + col;
    store4<T>(inter, gate_act_fast(a.act, g[0]) * u[0], gate_act_fast(a.act, g[1]) * u[1],
              gate_act_fast(a.act, g[2]) * u[2], gate_act_fast(a.act, g[3]) * u[3]);
  } else {
    float* y = static_cast<float*>(a.out) + static_cast<size_t>(split) * a.R * a.H +
               static_cast<size_t>(prow) * a.H + col;
    store4<float>(y, acc[0][0], acc[0][1], acc[0][2], acc[0][3]);
  }
}

template <bool kGateUp>
hipError_t launch_skinny(const FfnArgs& a, int dtype, hipStream_t s) {
  if (a.n_wtiles == 0 || a.max_tiles == 0) return hipSuccess;
  if (a.self_permute && (!kGateUp || a.perm.R > kWave)) return hipErrorInvalidValue;  // one wave groups
  const dim3 grid((a.n_wtiles + kWavesPerBlock - 1) / kWavesPerBlock, a.max_tiles, a.splits);
  if (a.self_permute) {
    if (dtype == MOE355_BF16)
      ffn_skinny_kernel<bf16, true, true><<<grid, dim3(kThreads), 0, s>>>(a);
    else
      ffn_skinny_kernel<f16, true, true><<<grid, dim3(kThreads), 0, s>>>(a);
  } else if (dtype == MOE355_BF16) {
    ffn_skinny_kernel<bf16, kGateUp, false><<<grid, dim3(kThreads), 0, s>>>(a);
  } else {
    ffn_skinny_kernel<f16, kGateUp, false><<<grid, dim3(kThreads), 0, s>>>(a);
  }
  return hipGetLastError();
}

}  // namespace

hipError_t launch_gate_up_skinny(const FfnArgs& a, int dtype, hipStream_t s) {
  return launch_skinny<true>(a, dtype, s);
}

hipError_t launch_down_skinny(const FfnArgs& a, int dtype, hipStream_t s) {
  return launch_skinny<false>(a, dtype, s);
}

}  // namespace moe355
