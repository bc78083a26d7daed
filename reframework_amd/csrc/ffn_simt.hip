// Grouped expert FFN with fp32 FMA tiles.
//
// Serves fp32 layers (the reference's fp32 model dtype, where the outputs must
// agree with fp32 arithmetic to 1e-5 relative, which rules out reduced-
// precision MFMA inputs) and shapes the MFMA kernels do not tile. Same
// contract as the tiled kernels (reframework/moe/fused.py:76-83): one launch
// over (64-feature tile) x (64-token tile) from the tile map, gather from x
// through row_src, gated activation fused into gate_up.
#include "common.h"

namespace moe355 {
namespace {

constexpr int kThreads = 256;
constexpr int kBN = 64;  // output features per tile
constexpr int kBT = 64;  // token rows per tile
constexpr int kBK = 16;

template <typename T, bool kGateUp>
__global__ __launch_bounds__(kThreads) void ffn_simt_kernel(const FfnArgs a) {
  constexpr int WR = kGateUp ? 2 * kBN : kBN;
  __shared__ float ws[kBK][WR + 4];
  __shared__ float xs[kBK][kBT + 4];

  const int tid = threadIdx.x, tx = tid & 15, ty = tid >> 4;
  const int wtile = blockIdx.x, ttile = blockIdx.y;
  if (ttile >= a.tile_map[0]) return;
  const int e = a.tile_map[2 + 2 * ttile];
  const int row0 = a.tile_map[3 + 2 * ttile];
  const int row_end = min(row0 + kBT, a.offsets[e + 1]);

  const int ld = kGateUp ? a.H : a.I;
  const int nout = kGateUp ? a.I : a.H;
  const int n0 = wtile * kBN;
  const T* w = static_cast<const T*>(a.w[e]);
  const T* x = static_cast<const T*>(a.x);

  float accg[4][4], accu[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) accg[i][j] = accu[i][j] = 0.f;

  for (int k0 = 0; k0 < ld; k0 += kBK) {
    for (int i = tid; i < WR * kBK; i += kThreads) {
      const int r = i / kBK, kk = i - r * kBK;
      const int feat = n0 + (kGateUp && r >= kBN ? r - kBN : r);
      const int wrow = kGateUp && r >= kBN ? a.I + feat : feat;
      const bool ok = feat < nout && k0 + kk < ld;
      ws[kk][r] = ok ? to_f32(w[static_cast<size_t>(wrow) * ld + k0 + kk]) : 0.f;
    }
    for (int i = tid; i < kBT * kBK; i += kThreads) {
      const int r = i / kBK, kk = i - r * kBK;
      const int prow = row0 + r;
      const bool ok = prow < row_end && k0 + kk < ld;
      float v = 0.f;
      if (ok) {
        const size_t xrow = kGateUp ? static_cast<size_t>(a.row_src[prow]) : static_cast<size_t>(prow);
        v = to_f32(x[xrow * ld + k0 + kk]);
      }
      xs[kk][r] = v;
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < kBK; ++kk) {
      float wv[4], uv[4], xv[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        wv[i] = ws[kk][tx + 16 * i];
        if (kGateUp) uv[i] = ws[kk][kBN + tx + 16 * i];
        xv[i] = xs[kk][ty + 16 * i];
      }
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          accg[i][j] = fmaf(wv[i], xv[j], accg[i][j]);
          if (kGateUp) accu[i][j] = fmaf(uv[i], xv[j], accu[i][j]);
        }
    }
    __syncthreads();
  }

#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int prow = row0 + ty + 16 * j;
    if (prow >= row_end) continue;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int feat = n0 + tx + 16 * i;
      if (feat >= nout) continue;
      if (kGateUp) {
        T* inter = static_cast<T*>(a.out);
        inter[static_cast<size_t>(prow) * a.I + feat] =
            from_f32<T>(gate_act(a.act, accg[i][j]) * accu[i][j]);
      } else {
        float* y = static_cast<float*>(a.out);
        y[static_cast<size_t>(prow) * a.H + feat] = accg[i][j];
      }
    }
  }
}

template <bool kGateUp>
hipError_t launch_simt(const FfnArgs& a, int dtype, hipStream_t s) {
  if (a.n_wtiles == 0 || a.max_tiles == 0) return hipSuccess;
  const dim3 grid(a.n_wtiles, a.max_tiles);
  if (dtype == MOE355_BF16)
    ffn_simt_kernel<bf16, kGateUp><<<grid, dim3(kThreads), 0, s>>>(a);
  else if (dtype == MOE355_F16)
    ffn_simt_kernel<f16, kGateUp><<<grid, dim3(kThreads), 0, s>>>(a);
  else
    ffn_simt_kernel<float, kGateUp><<<grid, dim3(kThreads), 0, s>>>(a);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_gate_up_simt(const FfnArgs& a, int dtype, hipStream_t s) {
  return launch_simt<true>(a, dtype, s);
}

hipError_t launch_down_simt(const FfnArgs& a, int dtype, hipStream_t s) {
  return launch_simt<false>(a, dtype, s);
}

}  // namespace moe355
