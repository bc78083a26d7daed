// Weighted combine back to token order, and the fp32 -> dtype cast.
//
// Replaces `y = y * w; out.index_add_(0, tok, y)` of fused_experts
// (reframework/moe/fused.py:84-86). Every token owns one workgroup and reads
// its K permuted rows (summing the down-projection K-splits on the way), so
// there are no atomics and the k order is fixed: results are deterministic.
// HBM bound: T*K*H*4*S bytes in, T*H*elem out.
#include "common.h"

namespace moe355 {
namespace {

constexpr int kThreads = 256;

template <typename OutT>
__global__ __launch_bounds__(kThreads) void combine_kernel(const CombineArgs a) {
  const int t = blockIdx.x;
  const size_t plane = static_cast<size_t>(a.R) * a.H;
  for (int h = threadIdx.x * 4; h < a.H; h += kThreads * 4) {
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    for (int k = 0; k < a.K; ++k) {
      const int row = a.slot_to_row[t * a.K + k];
      if (row < 0) continue;
      const float w = a.topk_w[t * a.K + k];
      const float* yr = a.y + static_cast<size_t>(row) * a.H + h;
      f32x4 ys = *reinterpret_cast<const f32x4*>(yr);
      for (int s = 1; s < a.splits; ++s) ys += *reinterpret_cast<const f32x4*>(yr + s * plane);
      acc += w * ys;
    }
    if (a.accumulate) {
      float* o = static_cast<float*>(a.out) + static_cast<size_t>(t) * a.H + h;
      *reinterpret_cast<f32x4*>(o) = *reinterpret_cast<const f32x4*>(o) + acc;
    } else {
      store4<OutT>(static_cast<OutT*>(a.out) + static_cast<size_t>(t) * a.H + h, acc[0], acc[1],
                   acc[2], acc[3]);
    }
  }
}

template <typename OutT>
__global__ __launch_bounds__(kThreads) void cast_kernel(const float* src, OutT* dst, size_t n) {
  for (size_t i = blockIdx.x * static_cast<size_t>(kThreads) + threadIdx.x; i < n;
       i += static_cast<size_t>(gridDim.x) * kThreads)
    dst[i] = from_f32<OutT>(src[i]);
}

}  // namespace

hipError_t launch_combine(const CombineArgs& a, int out_dtype, hipStream_t s) {
  if (a.T == 0) return hipSuccess;
  const dim3 grid(a.T), block(kThreads);
  if (a.accumulate || out_dtype == MOE355_F32)
    combine_kernel<float><<<grid, block, 0, s>>>(a);
  else if (out_dtype == MOE355_BF16)
    combine_kernel<bf16><<<grid, block, 0, s>>>(a);
  else
    combine_kernel<f16><<<grid, block, 0, s>>>(a);
  return hipGetLastError();
}

hipError_t launch_cast_f32(const float* src, void* dst, size_t n, int dtype, hipStream_t s) {
  if (n == 0) return hipSuccess;
  size_t blocks = (n + kThreads - 1) / kThreads;
  if (blocks > 65536) blocks = 65536;
  if (dtype == MOE355_BF16)
    cast_kernel<bf16><<<dim3(blocks), dim3(kThreads), 0, s>>>(src, static_cast<bf16*>(dst), n);
  else if (dtype == MOE355_F16)
    cast_kernel<f16><<<dim3(blocks), dim3(kThreads), 0, s>>>(src, static_cast<f16*>(dst), n);
  else
    cast_kernel<float><<<dim3(blocks), dim3(kThreads), 0, s>>>(src, static_cast<float*>(dst), n);
  return hipGetLastError();
}

}  // namespace moe355
