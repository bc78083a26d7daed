// Residual add + RMSNorm, the step before the MoE block in a decoder layer.
//
// Replaces RMSNorm._forward / forward_add_residual
// (reframework/layers/norm.py:27-53), called before the MoE at
// reframework/models/base.py:135:
//   residual = x + residual            (in the storage dtype)
//   normed   = residual * (1 / sqrt(mean(residual^2) + eps)) * w (+ b)
// computed in fp32 and rounded once to the storage dtype. One workgroup per
// token row keeps the row in registers between the sum of squares and the
// scaling, so the row is read once and each output written once: HBM bound,
// 2 * H * elem bytes read and 2 * H * elem written per row (1 + 1 without the
// residual add).
#include "common.h"

namespace moe355 {
namespace {

constexpr int kThreads = 256;
constexpr int kMaxChunks = 8;  // 16-byte chunks per thread: H <= 8 * 256 * (16 / elem)

template <typename T>
__device__ __forceinline__ u32x4 pack16(const float* v);

template <>
__device__ __forceinline__ u32x4 pack16<float>(const float* v) {
  return u32x4{__float_as_uint(v[0]), __float_as_uint(v[1]), __float_as_uint(v[2]),
               __float_as_uint(v[3])};
}

template <>
__device__ __forceinline__ u32x4 pack16<bf16>(const float* v) {
  bf16x8 h;
#pragma unroll
  for (int i = 0; i < 8; ++i) h[i] = from_f32<bf16>(v[i]);
  return __builtin_bit_cast(u32x4, h);
}

template <>
__device__ __forceinline__ u32x4 pack16<f16>(const float* v) {
  f16x8 h;
#pragma unroll
  for (int i = 0; i < 8; ++i) h[i] = from_f32<f16>(v[i]);
  return __builtin_bit_cast(u32x4, h);
}

// Weight / bias element e as fp32 (they may be stored in the layer dtype or fp32).
__device__ __forceinline__ float param_at(const void* p, int dtype, int e) {
  if (dtype == MOE355_F32) return static_cast<const float*>(p)[e];
  if (dtype == MOE355_BF16) return to_f32(static_cast<const bf16*>(p)[e]);
  return to_f32(static_cast<const f16*>(p)[e]);
}

template <typename T>
__global__ __launch_bounds__(kThreads) void add_rmsnorm_kernel(const NormArgs a) {
  constexpr int N = Vec16<T>::N;  // elements per 16-byte chunk
  const int t = blockIdx.x, tid = threadIdx.x;
  const int chunks = a.H / N;
  const size_t row = static_cast<size_t>(t) * a.H;
  __shared__ float red[kThreads / kWave];

  float r[kMaxChunks][N];
  float ss = 0.f;
#pragma unroll
  for (int c = 0; c < kMaxChunks; ++c) {
    const int ch = tid + c * kThreads;
    if (ch >= chunks) break;
    const size_t off = row + static_cast<size_t>(ch) * N;
    Vec16<T>::unpack(*reinterpret_cast<const u32x4*>(static_cast<const T*>(a.x) + off), r[c]);
    if (a.residual) {
      float s[N];
      Vec16<T>::unpack(*reinterpret_cast<const u32x4*>(static_cast<const T*>(a.residual) + off), s);
      // the sum is rounded to the storage dtype, as the reference adds there
#pragma unroll
      for (int i = 0; i < N; ++i) r[c][i] = to_f32(from_f32<T>(r[c][i] + s[i]));
      *reinterpret_cast<u32x4*>(static_cast<T*>(a.residual_out) + off) = pack16<T>(r[c]);
    }
#pragma unroll
    for (int i = 0; i < N; ++i) ss += r[c][i] * r[c][i];
  }
  ss = wave_sum(ss);
  if ((tid & (kWave - 1)) == 0) red[tid / kWave] = ss;
  __syncthreads();
  float tot = 0.f;
#pragma unroll
  for (int w = 0; w < kThreads / kWave; ++w) tot += red[w];
  const float inv = 1.0f / sqrtf(tot / static_cast<float>(a.H) + a.eps);

#pragma unroll
  for (int c = 0; c < kMaxChunks; ++c) {
    const int ch = tid + c * kThreads;
    if (ch >= chunks) break;
    float o[N];
#pragma unroll
    for (int i = 0; i < N; ++i) {
      const int e = ch * N + i;
      o[i] = r[c][i] * inv * param_at(a.weight, a.weight_dtype, e);
      if (a.bias) o[i] += param_at(a.bias, a.weight_dtype, e);
    }
    *reinterpret_cast<u32x4*>(static_cast<T*>(a.out) + row + static_cast<size_t>(ch) * N) =
        pack16<T>(o);
  }
}

}  // namespace

int norm_max_hidden(int dtype) {
  return kMaxChunks * kThreads * (dtype == MOE355_F32 ? 4 : 8);
}

hipError_t launch_add_rmsnorm(const NormArgs& a, int dtype, hipStream_t s) {
  if (a.T == 0) return hipSuccess;
  const dim3 grid(a.T), block(kThreads);
  if (dtype == MOE355_BF16)
    add_rmsnorm_kernel<bf16><<<grid, block, 0, s>>>(a);
  else if (dtype == MOE355_F16)
    add_rmsnorm_kernel<f16><<<grid, block, 0, s>>>(a);
  else
    add_rmsnorm_kernel<float><<<grid, block, 0, s>>>(a);
  return hipGetLastError();
}

}  // namespace moe355
