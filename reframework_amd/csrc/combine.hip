// Weighted combine back to token order, and the fp32 -> dtype cast.
//
// Replaces `y = y * w; out.index_add_(0, tok, y)` of fused_experts
// (reframework/moe/fused.py:84-86). Every token owns one workgroup and reads
// its K permuted rows (summing the down-projection K-splits on the way), so
// there are no atomics and the k order is fixed: results are deterministic.
// HBM bound: T*K*H*4*S bytes in (T*K*H*elem when y is in the layer dtype),
// T*H*elem out.
#include "common.h"

namespace moe355 {
namespace {

constexpr int kThreads = 256;

// Four consecutive y elements as fp32.
template <typename Y>
__device__ __forceinline__ f32x4 load4(const Y* p) {
  const u32x2 v = *reinterpret_cast<const u32x2*>(p);
  float o[8];
  Vec16<Y>::unpack(u32x4{v.x, v.y, 0u, 0u}, o);
  return f32x4{o[0], o[1], o[2], o[3]};
}

template <>
__device__ __forceinline__ f32x4 load4<float>(const float* p) {
  return *reinterpret_cast<const f32x4*>(p);
}

// Workgroup (t, hb) produces out[t, hb*1024 .. +1024): each thread one group
// of 4 features. The K slots' rows and weights are uniform per workgroup; the
// S split partials of every slot are issued as independent loads, so a
// decode-size combine costs one round trip, not S*K of them. Y is fp32 for
// split partials, or the layer dtype (one split, y16).
template <typename OutT, typename Y, int S>
__global__ __launch_bounds__(kThreads) void combine_kernel(const CombineArgs a) {
  const int t = blockIdx.x;
  const int h = (blockIdx.y * kThreads + threadIdx.x) * 4;
  if (h >= a.H) return;
  const size_t plane = static_cast<size_t>(a.R) * a.H;
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  for (int k = 0; k < a.K; ++k) {
    const int row = a.slot_to_row[t * a.K + k];
    if (row < 0) continue;
    const float w = a.topk_w[t * a.K + k];
    const Y* yr = static_cast<const Y*>(a.y) + static_cast<size_t>(row) * a.H + h;
    f32x4 part[S];
#pragma unroll
    for (int s = 0; s < S; ++s) part[s] = load4<Y>(yr + s * plane);
    f32x4 ys = part[0];
#pragma unroll
    for (int s = 1; s < S; ++s) ys += part[s];
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

template <typename OutT>
__global__ __launch_bounds__(kThreads) void cast_kernel(const float* src, OutT* dst, size_t n) {
  for (size_t i = blockIdx.x * static_cast<size_t>(kThreads) + threadIdx.x; i < n;
       i += static_cast<size_t>(gridDim.x) * kThreads)
    dst[i] = from_f32<OutT>(src[i]);
}

template <typename OutT>
hipError_t launch_combine_t(const CombineArgs& a, int dtype, hipStream_t s) {
  const dim3 grid(a.T, (a.H + kThreads * 4 - 1) / (kThreads * 4)), block(kThreads);
  if (a.y16) {
    if (a.splits != 1 || dtype == MOE355_F32) return hipErrorInvalidValue;
    if (dtype == MOE355_BF16)
      combine_kernel<OutT, bf16, 1><<<grid, block, 0, s>>>(a);
    else
      combine_kernel<OutT, f16, 1><<<grid, block, 0, s>>>(a);
    return hipGetLastError();
  }
  switch (a.splits) {
    case 1: combine_kernel<OutT, float, 1><<<grid, block, 0, s>>>(a); break;
    case 2: combine_kernel<OutT, float, 2><<<grid, block, 0, s>>>(a); break;
    case 4: combine_kernel<OutT, float, 4><<<grid, block, 0, s>>>(a); break;
    case 8: combine_kernel<OutT, float, 8><<<grid, block, 0, s>>>(a); break;
    case 16: combine_kernel<OutT, float, 16><<<grid, block, 0, s>>>(a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace

// out_dtype is the layer dtype (the type of y when a.y16).
hipError_t launch_combine(const CombineArgs& a, int out_dtype, hipStream_t s) {
  if (a.T == 0) return hipSuccess;
  if (a.accumulate || out_dtype == MOE355_F32) return launch_combine_t<float>(a, out_dtype, s);
  if (out_dtype == MOE355_BF16) return launch_combine_t<bf16>(a, out_dtype, s);
  return launch_combine_t<f16>(a, out_dtype, s);
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
