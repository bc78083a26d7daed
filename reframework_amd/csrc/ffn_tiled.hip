// Grouped expert FFN on bf16/f16 MFMA, prefill-sized groups.
//
// Replaces the per-expert GEMMs of fused_experts (reframework/moe/fused.py:
// 76-83): `x @ w1[e].t()`, gated_act_and_mul, `inter @ w2[e].t()`. One launch
// covers every expert: the grid is (weight tile) x (token tile) over the tile
// map written by the permute, so no host round trip decides group sizes.
//
// Tile: 256 weight rows x 256 token rows x 64 k per LDS stage, 4 waves in a
// 2x2 arrangement, each wave owning 4x4 blocks of v_mfma_f32_32x32x16 (a
// 128x128 sub-tile, 256 fp32 accumulators). Weight rows are the MFMA M side and
// tokens the N side, so each lane ends up holding 4 consecutive output features
// of one token and stores them as one vector.
//   gate_up: the 256 weight rows are 128 gate rows and the 128 matching up rows,
//            so gate and up of the same (token, feature) land in the same lane
//            and silu(g)*u is applied in registers; token rows are gathered
//            straight from x through row_src (no permuted copy of x).
//   down:    256 rows of w2 against the permuted inter rows, fp32 partials
//            per K-split into y.
// LDS rows are 128 B, XOR-swizzled in 16-byte chunks (swz) so that the staging
// writes and the MFMA operand reads are bank-conflict free. Global loads are
// staged through registers and double-buffered in LDS (2 x 64 KB).
#include "common.h"

namespace moe355 {
namespace {

constexpr int kThreads = 256;
constexpr int kTileW = 256;
constexpr int kTileT = 256;
constexpr int kBK = 64;
constexpr int kRowBytes = kBK * 2;
constexpr int kRowsPerPass = kThreads / 8;            // 8 threads x 16 B per row
constexpr int kPasses = kTileW / kRowsPerPass;        // 8
constexpr int kRegionBytes = kTileW * kRowBytes;      // 32 KB
constexpr int kStageBytes = 2 * kRegionBytes;         // weights + tokens
constexpr int kLdsBytes = 2 * kStageBytes;            // double buffered

// Physical 16-byte chunk of logical chunk c in LDS row r. Rows are 128 B (8
// chunks). XOR with r&7 spreads 8 consecutive rows over all 8 chunk columns,
// and the extra bit (r>>3)&1 keeps rows r and r+8, which share a bank set on a
// 64-bank LDS, in different columns: any 16 consecutive rows read at one
// logical chunk hit 16 distinct 16-byte bank groups.
__device__ __forceinline__ uint32_t swz(int c, int r) {
  return static_cast<uint32_t>(c ^ (r & 7) ^ ((r >> 3) & 1));
}

template <typename T>
struct Mfma32;

template <>
struct Mfma32<bf16> {
  __device__ __forceinline__ static f32x16 mma(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
};

template <>
struct Mfma32<f16> {
  __device__ __forceinline__ static f32x16 mma(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
};

template <typename T, bool kGateUp>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(1, 1)))
void ffn_tiled_kernel(const FfnArgs a) {
  __shared__ __attribute__((aligned(16))) uint8_t lds[kLdsBytes];

  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave;
  const int wave_w = wave >> 1, wave_t = wave & 1;

  const int L = xcd_remap(blockIdx.x, gridDim.x);
  const int per_split = a.n_wtiles * a.max_tiles;
  const int split = L / per_split;
  const int rem = L - split * per_split;
  const int wtile = rem / a.max_tiles;
  const int ttile = rem - wtile * a.max_tiles;
  if (ttile >= a.tile_map[0]) return;
  const int e = a.tile_map[2 + 2 * ttile];
  const int row0 = a.tile_map[3 + 2 * ttile];
  const int row_end = min(row0 + kTileT, a.offsets[e + 1]);

  const int ld = kGateUp ? a.H : a.I;  // elements per weight row and per token row
  const int kbeg = split * a.k_per_split;
  const int nk = a.k_per_split / kBK;

  const char* wbase = static_cast<const char*>(a.w[e]) + static_cast<size_t>(kbeg) * 2;
  const char* xbase = static_cast<const char*>(a.x) + static_cast<size_t>(kbeg) * 2;
  if (!kGateUp) xbase += static_cast<size_t>(row0) * ld * 2;

  // Byte offsets of this thread's 16-byte chunk in each of the 8 load passes.
  const int lrow = tid >> 3, chunk = tid & 7;
  uint32_t woff[kPasses], xoff[kPasses];
#pragma unroll
  for (int p = 0; p < kPasses; ++p) {
    const int r = p * kRowsPerPass + lrow;
    int wrow;
    if (kGateUp)
      wrow = r < kTileW / 2 ? wtile * (kTileW / 2) + r : a.I + wtile * (kTileW / 2) + (r - kTileW / 2);
    else
      wrow = wtile * kTileW + r;
    woff[p] = static_cast<uint32_t>(wrow) * static_cast<uint32_t>(ld * 2) + chunk * 16;
    const int prow = min(row0 + r, row_end - 1);
    const int xrow = kGateUp ? a.row_src[prow] : prow - row0;
    xoff[p] = static_cast<uint32_t>(xrow) * static_cast<uint32_t>(ld * 2) + chunk * 16;
  }
  const uint32_t st_off = lrow * kRowBytes + (swz(chunk, lrow) << 4);

  // MFMA operand rows of this wave inside the stage.
  const int lr = lane & 31, kh = lane >> 5;
  uint32_t arow[4], brow[4];
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    int rb;
    if (kGateUp)
      rb = b < 2 ? wave_w * 64 + b * 32 : kTileW / 2 + wave_w * 64 + (b - 2) * 32;
    else
      rb = wave_w * 128 + b * 32;
    arow[b] = (rb + lr) * kRowBytes;
    brow[b] = kRegionBytes + (wave_t * 128 + b * 32 + lr) * kRowBytes;
  }
  // Swizzled 16-byte chunk offsets of the 4 k16 sub-steps for this lane
  // (operand rows start at multiples of 32, so row bits 0..3 are lr's).
  uint32_t coff[kBK / 16];
#pragma unroll
  for (int ks = 0; ks < kBK / 16; ++ks) coff[ks] = swz(ks * 2 + kh, lr) << 4;

  f32x16 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x16{};

  u32x4 wr[kPasses], xr[kPasses];
  auto load_stage = [&](int kt) {
    const char* wk = wbase + kt * kRowBytes;
    const char* xk = xbase + kt * kRowBytes;
#pragma unroll
    for (int p = 0; p < kPasses; ++p) {
      wr[p] = *reinterpret_cast<const u32x4*>(wk + woff[p]);
      xr[p] = *reinterpret_cast<const u32x4*>(xk + xoff[p]);
    }
  };
  auto store_stage = [&](int s) {
    uint8_t* st = lds + s * kStageBytes;
#pragma unroll
    for (int p = 0; p < kPasses; ++p) {
      *reinterpret_cast<u32x4*>(st + p * kRowsPerPass * kRowBytes + st_off) = wr[p];
      *reinterpret_cast<u32x4*>(st + kRegionBytes + p * kRowsPerPass * kRowBytes + st_off) = xr[p];
    }
  };
  auto read_frags = [&](const uint8_t* st, int ks, u32x4* af, u32x4* bf) {
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      af[b] = *reinterpret_cast<const u32x4*>(st + arow[b] + coff[ks]);
      bf[b] = *reinterpret_cast<const u32x4*>(st + brow[b] + coff[ks]);
    }
  };

  // Pipeline: LDS stage kt is consumed while stage kt+1 (already in
  // registers) is written to the other LDS buffer during sub-step 1, one LDS
  // write and one global load of stage kt+2 (clamped to the last stage, so the
  // loop has no branches) between consecutive MFMAs. Operand fragments of
  // sub-step ks+1 are read while sub-step ks's 16 MFMAs run; scheduling
  // fences keep the compiler from pulling those reads in front of the MFMAs
  // they are meant to overlap. One barrier per stage.
  load_stage(0);
  store_stage(0);
  load_stage(min(1, nk - 1));
  __syncthreads();

  for (int kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1;
    const uint8_t* st = lds + cur * kStageBytes;
    u32x4 fa[2][4], fb[2][4];
    read_frags(st, 0, fa[0], fb[0]);
#pragma unroll
    for (int ks = 0; ks < kBK / 16; ++ks) {
      if (ks + 1 < kBK / 16) read_frags(st, ks + 1, fa[(ks + 1) & 1], fb[(ks + 1) & 1]);
      __builtin_amdgcn_sched_barrier(0);
      if (ks == 1) {
        store_stage(cur ^ 1);
        load_stage(min(kt + 2, nk - 1));
      }
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          acc[i][j] = Mfma32<T>::mma(fa[ks & 1][i], fb[ks & 1][j], acc[i][j]);
      if (ks == 1) {
        for (int q = 0; q < 16; ++q) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
          __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);
          __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    __syncthreads();
  }

  // Epilogue. Lane (lr, kh) of block (i, j) holds, for q = 0..3, features
  // 8q + 4kh + 0..3 of the 32-row weight block and token lr of the token block.
  if (kGateUp) {
    T* inter = static_cast<T*>(a.out);
#pragma unroll
    for (int b = 0; b < 2; ++b) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int prow = row0 + wave_t * 128 + j * 32 + lr;
        if (prow < row_end) {
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const int col = wtile * (kTileW / 2) + wave_w * 64 + b * 32 + 8 * q + 4 * kh;
            float v[4];
#pragma unroll
            for (int r = 0; r < 4; ++r)
              v[r] = gate_act(a.act, acc[b][j][4 * q + r]) * acc[b + 2][j][4 * q + r];
            store4<T>(inter + static_cast<size_t>(prow) * a.I + col, v[0], v[1], v[2], v[3]);
          }
        }
      }
    }
  } else {
    float* y = static_cast<float*>(a.out) + static_cast<size_t>(split) * a.R * a.H;
#pragma unroll
    for (int b = 0; b < 4; ++b) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int prow = row0 + wave_t * 128 + j * 32 + lr;
        if (prow < row_end) {
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const int h = wtile * kTileW + wave_w * 128 + b * 32 + 8 * q + 4 * kh;
            store4<float>(y + static_cast<size_t>(prow) * a.H + h, acc[b][j][4 * q],
                          acc[b][j][4 * q + 1], acc[b][j][4 * q + 2], acc[b][j][4 * q + 3]);
          }
        }
      }
    }
  }
}

template <bool kGateUp>
hipError_t launch_tiled(const FfnArgs& a, int dtype, hipStream_t s) {
  const int nwg = a.n_wtiles * a.max_tiles * a.splits;
  if (nwg == 0) return hipSuccess;
  if (dtype == MOE355_BF16)
    ffn_tiled_kernel<bf16, kGateUp><<<dim3(nwg), dim3(kThreads), 0, s>>>(a);
  else
    ffn_tiled_kernel<f16, kGateUp><<<dim3(nwg), dim3(kThreads), 0, s>>>(a);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_gate_up_tiled(const FfnArgs& a, int dtype, hipStream_t s) {
  return launch_tiled<true>(a, dtype, s);
}

hipError_t launch_down_tiled(const FfnArgs& a, int dtype, hipStream_t s) {
  return launch_tiled<false>(a, dtype, s);
}

}  // namespace moe355
