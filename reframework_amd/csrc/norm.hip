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

// N consecutive weight / bias elements stored as W, read with 16-byte (or, for
// 4 elements of a 16-bit type, 8-byte) vector loads.
template <typename W, int N>
struct ParamChunk {
  static constexpr int kBytes = N * static_cast<int>(sizeof(W));
  static constexpr int kVecs = kBytes >= 16 ? kBytes / 16 : 1;
  u32x4 raw[kVecs];

  __device__ __forceinline__ void load(const W* p, int e0) {
    if constexpr (kBytes >= 16) {
#pragma unroll
      for (int i = 0; i < kVecs; ++i)
        raw[i] = *reinterpret_cast<const u32x4*>(p + e0 + i * (16 / static_cast<int>(sizeof(W))));
    } else {
      const u32x2 t = *reinterpret_cast<const u32x2*>(p + e0);
      raw[0] = u32x4{t.x, t.y, 0u, 0u};
    }
  }

  __device__ __forceinline__ void unpack(float* o) const {
    const uint32_t* w = reinterpret_cast<const uint32_t*>(raw);
#pragma unroll
    for (int i = 0; i < N; ++i) {
      if constexpr (sizeof(W) == 4) {
        o[i] = __uint_as_float(w[i]);
      } else {
        const uint32_t h = (w[i / 2] >> (16 * (i & 1))) & 0xffffu;
        if constexpr (std::is_same<W, bf16>::value)
          o[i] = __uint_as_float(h << 16);
        else
          o[i] = static_cast<float>(__builtin_bit_cast(f16, static_cast<uint16_t>(h)));
      }
    }
  }
};

// One workgroup per row; thread tid owns 16-byte chunks tid, tid + 256, ...
// (CPT of them at most). Every load of a phase is issued before any is used:
// phase 1 reads x and the residual, phase 2 (after the sum of squares) the
// weight and bias, so each phase costs one memory round trip.
template <typename T, typename W, int CPT>
__global__ __launch_bounds__(kThreads) void add_rmsnorm_kernel(const NormArgs a) {
  constexpr int N = Vec16<T>::N;  // elements per 16-byte chunk
  const int t = blockIdx.x, tid = threadIdx.x;
  const int chunks = a.H / N;
  const size_t row = static_cast<size_t>(t) * a.H;
  __shared__ float red[kThreads / kWave];
  const T* xr = static_cast<const T*>(a.x) + row;
  const T* rr = static_cast<const T*>(a.residual) + row;

  u32x4 xraw[CPT], rraw[CPT];
#pragma unroll
  for (int c = 0; c < CPT; ++c) {
    const int ch = tid + c * kThreads;
    if (ch < chunks) {
      xraw[c] = *reinterpret_cast<const u32x4*>(xr + static_cast<size_t>(ch) * N);
      if (a.residual) rraw[c] = *reinterpret_cast<const u32x4*>(rr + static_cast<size_t>(ch) * N);
    }
  }
  float r[CPT][N];
  float ss = 0.f;
#pragma unroll
  for (int c = 0; c < CPT; ++c) {
    const int ch = tid + c * kThreads;
    if (ch >= chunks) continue;
    Vec16<T>::unpack(xraw[c], r[c]);
    if (a.residual) {
      float s[N];
      Vec16<T>::unpack(rraw[c], s);
      // the sum is rounded to the storage dtype, as the reference adds there
#pragma unroll
      for (int i = 0; i < N; ++i) r[c][i] = to_f32(from_f32<T>(r[c][i] + s[i]));
      *reinterpret_cast<u32x4*>(static_cast<T*>(a.residual_out) + row + static_cast<size_t>(ch) * N) =
          pack16<T>(r[c]);
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

  ParamChunk<W, N> wc[CPT], bc[CPT];
#pragma unroll
  for (int c = 0; c < CPT; ++c) {
    const int ch = tid + c * kThreads;
    if (ch < chunks) {
      wc[c].load(static_cast<const W*>(a.weight), ch * N);
      if (a.bias) bc[c].load(static_cast<const W*>(a.bias), ch * N);
    }
  }
#pragma unroll
  for (int c = 0; c < CPT; ++c) {
    const int ch = tid + c * kThreads;
    if (ch >= chunks) continue;
    float wv[N], bv[N];
    wc[c].unpack(wv);
    if (a.bias) bc[c].unpack(bv);
    float o[N];
#pragma unroll
    for (int i = 0; i < N; ++i) {
      o[i] = r[c][i] * inv * wv[i];
      if (a.bias) o[i] += bv[i];
    }
    *reinterpret_cast<u32x4*>(static_cast<T*>(a.out) + row + static_cast<size_t>(ch) * N) =
        pack16<T>(o);
  }
}

template <typename T, typename W>
hipError_t launch_norm_tw(const NormArgs& a, hipStream_t s) {
  const int per_thread = (a.H / Vec16<T>::N + kThreads - 1) / kThreads;
  const dim3 grid(a.T), block(kThreads);
  if (per_thread <= 1)
    add_rmsnorm_kernel<T, W, 1><<<grid, block, 0, s>>>(a);
  else if (per_thread <= 2)
    add_rmsnorm_kernel<T, W, 2><<<grid, block, 0, s>>>(a);
  else if (per_thread <= 4)
    add_rmsnorm_kernel<T, W, 4><<<grid, block, 0, s>>>(a);
  else
    add_rmsnorm_kernel<T, W, kMaxChunks><<<grid, block, 0, s>>>(a);
  return hipGetLastError();
}

template <typename T>
hipError_t launch_norm_t(const NormArgs& a, hipStream_t s) {
  if (a.weight_dtype == MOE355_BF16) return launch_norm_tw<T, bf16>(a, s);
  if (a.weight_dtype == MOE355_F16) return launch_norm_tw<T, f16>(a, s);
  return launch_norm_tw<T, float>(a, s);
}

}  // namespace

int norm_max_hidden(int dtype) {
  return kMaxChunks * kThreads * (dtype == MOE355_F32 ? 4 : 8);
}

hipError_t launch_add_rmsnorm(const NormArgs& a, int dtype, hipStream_t s) {
  if (a.T == 0) return hipSuccess;
  if (dtype == MOE355_BF16) return launch_norm_t<bf16>(a, s);
  if (dtype == MOE355_F16) return launch_norm_t<f16>(a, s);
  return launch_norm_t<float>(a, s);
}

}  // namespace moe355
