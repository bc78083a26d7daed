// Grouped expert FFN for decode-sized groups (a few tokens per expert).
//
// Replaces the same per-expert GEMMs as the tiled kernel
// (reframework/moe/fused.py:76-83) when each expert sees <= 16-ish rows. Then
// the layer is a weight stream: every routed expert's 3*H*I weights are read
// once and each weight meets only a handful of tokens, so the kernel is built
// for HBM bandwidth, not for MFMA reuse.
//
// Each wave owns 16 weight rows (gate_up: 16 gate rows + the 16 matching up
// rows) of one expert and one 16-token tile, and walks K in 32-element steps
// with v_mfma_f32_16x16x32 (weights on the M side, tokens on the N side). The
// weight operand is loaded from HBM straight into the MFMA registers: lane l
// reads 16 bytes of row l%16 at k offset 8*(l/16), so a wave step touches 64
// contiguous bytes of each of 16 rows and consecutive steps finish the 128-byte
// lines. Loads are unrolled 8 steps deep so every wave keeps 16-24 KB in
// flight; with several waves per SIMD the CU sustains the HBM stream without
// LDS. The token operand (a few KB per expert) is re-read from L1/L2.
// gate_up fuses the gated activation; down writes fp32 partials per K-split,
// which the combine kernel sums, so the short down projection of a decode step
// still spreads over every CU.
#include "common.h"

namespace moe355 {
namespace {

constexpr int kThreads = 256;
constexpr int kWavesPerBlock = kThreads / kWave;
constexpr int kRows = 16;
constexpr int kStep = 32;
constexpr int kUnroll = 8;

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

template <typename T, bool kGateUp>
__global__ __launch_bounds__(kThreads) void ffn_skinny_kernel(const FfnArgs a) {
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
  const int group = blockIdx.x * kWavesPerBlock + wave;
  const int ttile = blockIdx.y, split = blockIdx.z;
  if (ttile >= a.tile_map[0] || group >= a.n_wtiles) return;
  const int e = a.tile_map[2 + 2 * ttile];
  const int row0 = a.tile_map[3 + 2 * ttile];
  const int row_end = min(row0 + kRows, a.offsets[e + 1]);

  const int lr = lane & 15, kq = lane >> 4;
  const int ld = kGateUp ? a.H : a.I;
  const int kbeg = split * a.k_per_split;
  const int kend = kbeg + a.k_per_split;

  const T* w = static_cast<const T*>(a.w[e]);
  const T* wg = w + static_cast<size_t>(group * kRows + lr) * ld + kq * 8;
  const T* wu = kGateUp ? w + static_cast<size_t>(a.I + group * kRows + lr) * ld + kq * 8 : wg;
  const int prow = row0 + lr;
  const bool valid = prow < row_end;
  const int xrow = kGateUp ? a.row_src[valid ? prow : row0] : (valid ? prow : row0);
  const T* xp = static_cast<const T*>(a.x) + static_cast<size_t>(xrow) * ld + kq * 8;
  const u32x4 zero = {0, 0, 0, 0};

  f32x4 accg = {0.f, 0.f, 0.f, 0.f}, accu = {0.f, 0.f, 0.f, 0.f};
  int k = kbeg;
  for (; k + kUnroll * kStep <= kend; k += kUnroll * kStep) {
    u32x4 g[kUnroll], u[kUnroll], xv[kUnroll];
#pragma unroll
    for (int i = 0; i < kUnroll; ++i) {
      g[i] = load16_stream(wg + k + i * kStep);
      if (kGateUp) u[i] = load16_stream(wu + k + i * kStep);
      xv[i] = valid ? load16(xp + k + i * kStep) : zero;
    }
#pragma unroll
    for (int i = 0; i < kUnroll; ++i) {
      accg = Mfma16<T>::mma(g[i], xv[i], accg);
      if (kGateUp) accu = Mfma16<T>::mma(u[i], xv[i], accu);
    }
  }
  for (; k + kStep <= kend; k += kStep) {
    const u32x4 g = load16_stream(wg + k);
    const u32x4 xv = valid ? load16(xp + k) : zero;
    accg = Mfma16<T>::mma(g, xv, accg);
    if (kGateUp) {
      const u32x4 u = load16_stream(wu + k);
      accu = Mfma16<T>::mma(u, xv, accu);
    }
  }

  // Lane (lr, kq) holds features 4*kq + 0..3 of this 16-row group for token lr.
  if (!valid) return;
  const int col = group * kRows + 4 * kq;
  if (kGateUp) {
    T* inter = static_cast<T*>(a.out) + static_cast<size_t>(prow) * a.I + col;
    store4<T>(inter, gate_act(a.act, accg[0]) * accu[0], gate_act(a.act, accg[1]) * accu[1],
              gate_act(a.act, accg[2]) * accu[2], gate_act(a.act, accg[3]) * accu[3]);
  } else {
    float* y = static_cast<float*>(a.out) + static_cast<size_t>(split) * a.R * a.H +
               static_cast<size_t>(prow) * a.H + col;
    store4<float>(y, accg[0], accg[1], accg[2], accg[3]);
  }
}

template <bool kGateUp>
hipError_t launch_skinny(const FfnArgs& a, int dtype, hipStream_t s) {
  if (a.n_wtiles == 0 || a.max_tiles == 0) return hipSuccess;
  const dim3 grid((a.n_wtiles + kWavesPerBlock - 1) / kWavesPerBlock, a.max_tiles, a.splits);
  if (dtype == MOE355_BF16)
    ffn_skinny_kernel<bf16, kGateUp><<<grid, dim3(kThreads), 0, s>>>(a);
  else
    ffn_skinny_kernel<f16, kGateUp><<<grid, dim3(kThreads), 0, s>>>(a);
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
