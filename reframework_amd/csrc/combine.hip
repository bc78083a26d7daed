// Weighted combine back to token order, and the fp32 -> dtype cast.
//
// Replaces `y = y * w; out.index_add_(0, tok, y)` of fused_experts
// (reframework/moe/fused.py:84-86). Each workgroup covers a slice of one
// token's features and reads that slice of its K permuted rows (summing the
// down-projection K-splits on the way), so there are no atomics and the k
// order is fixed: results are deterministic.
// HBM bound: T*K*H*4*S bytes in (T*K*H*elem when y is in the layer dtype),
// T*H*elem out.
#include "common.h"

namespace moe355 {
namespace {

constexpr int kThreads = 256;

// V consecutive y elements (4 or 8) as fp32: 8 or 16 bytes of a 16-bit y,
// one or two 16-byte loads of fp32 partials.
template <typename Y, int V>
__device__ __forceinline__ void loadv(const Y* p, float* o) {
  if constexpr (std::is_same<Y, float>::value) {
#pragma unroll
    for (int i = 0; i < V; i += 4) {
      const f32x4 v = *reinterpret_cast<const f32x4*>(p + i);
      o[i] = v[0];
      o[i + 1] = v[1];
      o[i + 2] = v[2];
      o[i + 3] = v[3];
    }
  } else if constexpr (V == 8) {
    Vec16<Y>::unpack(*reinterpret_cast<const u32x4*>(p), o);
  } else {
    const u32x2 v = *reinterpret_cast<const u32x2*>(p);
    float t[8];
    Vec16<Y>::unpack(u32x4{v.x, v.y, 0u, 0u}, t);
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = t[i];
  }
}

template <typename OutT, int V>
__device__ __forceinline__ void storev(OutT* p, const float* v) {
#pragma unroll
  for (int i = 0; i < V; i += 4) store4<OutT>(p + i, v[i], v[i + 1], v[i + 2], v[i + 3]);
}

// Workgroup (t, hb) of NT threads produces out[t, hb*NT*V .. +NT*V), V
// features per thread. The K slots' rows and weights are uniform per
// workgroup. Slots go in batches of KB: every load of a batch (its slots'
// S split partials) is issued before the first is used, so a token costs one
// memory round trip per batch, not one per slot and split; a dropped slot
// (row -1) loads row 0 and its values are discarded by a select (not scaled by
// a zero weight, which would turn an inf in row 0 into a NaN). Slots, and the
// splits of each slot, are summed in ascending order. Y is fp32 for split
// partials, or the layer dtype (one split, y16).
template <typename OutT, typename Y, int S, int V, int NT>
__global__ __launch_bounds__(NT) void combine_kernel(const CombineArgs a) {
  constexpr int KB = S >= 16 ? 1 : S >= 8 ? 2 : S >= 4 ? 4 : 8;
  const int t = blockIdx.x;
  const int h = (blockIdx.y * NT + threadIdx.x) * V;
  if (h >= a.H) return;
  const size_t plane = static_cast<size_t>(a.R) * a.H;
  const int* s2r = a.slot_to_row + static_cast<size_t>(t) * a.K;
  const float* tw = a.topk_w + static_cast<size_t>(t) * a.K;
  float acc[V];
#pragma unroll
  for (int i = 0; i < V; ++i) acc[i] = 0.f;
  for (int k0 = 0; k0 < a.K; k0 += KB) {
    int row[KB];
    float w[KB];
#pragma unroll
    for (int j = 0; j < KB; ++j) {
      row[j] = k0 + j < a.K ? s2r[k0 + j] : -1;
      w[j] = k0 + j < a.K ? tw[k0 + j] : 0.f;
    }
    float part[KB][S][V];
#pragma unroll
    for (int j = 0; j < KB; ++j) {
      const Y* yr = static_cast<const Y*>(a.y) + static_cast<size_t>(row[j] < 0 ? 0 : row[j]) * a.H + h;
#pragma unroll
      for (int s = 0; s < S; ++s) loadv<Y, V>(yr + s * plane, part[j][s]);
    }
#pragma unroll
    for (int j = 0; j < KB; ++j) {
      if (row[j] < 0) continue;
#pragma unroll
      for (int i = 0; i < V; ++i) {
        float ys = part[j][0][i];
#pragma unroll
        for (int s = 1; s < S; ++s) ys += part[j][s][i];
        acc[i] += w[j] * ys;
      }
    }
  }
  if (a.accumulate) {
    float* o = static_cast<float*>(a.out) + static_cast<size_t>(t) * a.H + h;
    float prev[V];
    loadv<float, V>(o, prev);
#pragma unroll
    for (int i = 0; i < V; ++i) prev[i] += acc[i];
    storev<float, V>(o, prev);
  } else {
    storev<OutT, V>(static_cast<OutT*>(a.out) + static_cast<size_t>(t) * a.H + h, acc);
  }
}

// Prefill sizes with one y plane (one split) and K <= KM slots per token:
// workgroup (tb, hb) produces out[t, hb*2048 .. +2048) for the TPB tokens
// t = tb*TPB .. +TPB, 8 features per thread, and issues the loads of all
// TPB*KM rows before the first is used. One token per workgroup kept only its
// K rows (8 KB at K = 2) in flight per memory round trip and ran at ~5 TB/s.
// Slot reads past K or past the last token are clamped in bounds and their
// rows treated as dropped. Sums run over a token's slots in ascending order,
// as in combine_kernel.
template <typename OutT, typename Y, int KM, int TPB>
__global__ __launch_bounds__(kThreads) void combine_tokens_kernel(const CombineArgs a) {
  constexpr int V = 8;
  const int h = (blockIdx.y * kThreads + threadIdx.x) * V;
  if (h >= a.H) return;
  const int t0 = blockIdx.x * TPB;
  int row[TPB][KM];
  float w[TPB][KM];
#pragma unroll
  for (int tt = 0; tt < TPB; ++tt) {
    const int tc = min(t0 + tt, a.T - 1);
#pragma unroll
    for (int j = 0; j < KM; ++j) {
      const size_t slot = static_cast<size_t>(tc) * a.K + min(j, a.K - 1);
      const bool ok = j < a.K && t0 + tt < a.T;
      const int r = a.slot_to_row[slot];
      const float wt = a.topk_w[slot];
      row[tt][j] = ok ? r : -1;
      w[tt][j] = ok ? wt : 0.f;
    }
  }
  float part[TPB][KM][V];
#pragma unroll
  for (int tt = 0; tt < TPB; ++tt)
#pragma unroll
    for (int j = 0; j < KM; ++j)
      loadv<Y, V>(static_cast<const Y*>(a.y) +
                      static_cast<size_t>(row[tt][j] < 0 ? 0 : row[tt][j]) * a.H + h,
                  part[tt][j]);
#pragma unroll
  for (int tt = 0; tt < TPB; ++tt) {
    if (t0 + tt >= a.T) break;
    float acc[V];
#pragma unroll
    for (int i = 0; i < V; ++i) acc[i] = 0.f;
#pragma unroll
    for (int j = 0; j < KM; ++j) {
      if (row[tt][j] < 0) continue;
#pragma unroll
      for (int i = 0; i < V; ++i) acc[i] += w[tt][j] * part[tt][j][i];
    }
    const size_t o = static_cast<size_t>(t0 + tt) * a.H + h;
    if (a.accumulate) {
      float prev[V];
      loadv<float, V>(static_cast<float*>(a.out) + o, prev);
#pragma unroll
      for (int i = 0; i < V; ++i) prev[i] += acc[i];
      storev<float, V>(static_cast<float*>(a.out) + o, prev);
    } else {
      storev<OutT, V>(static_cast<OutT*>(a.out) + o, acc);
    }
  }
}

template <typename OutT, typename Y, int KM>
hipError_t launch_combine_tokens(const CombineArgs& a, hipStream_t s) {
  constexpr int TPB = 16 / KM < 4 ? 16 / KM : 4;  // 8-16 rows in flight per workgroup
  const dim3 grid((a.T + TPB - 1) / TPB, (a.H + kThreads * 8 - 1) / (kThreads * 8));
  combine_tokens_kernel<OutT, Y, KM, TPB><<<grid, dim3(kThreads), 0, s>>>(a);
  return hipGetLastError();
}

template <typename OutT, typename Y>
hipError_t launch_combine_tokens_k(const CombineArgs& a, hipStream_t s) {
  if (a.K <= 1) return launch_combine_tokens<OutT, Y, 1>(a, s);
  if (a.K <= 2) return launch_combine_tokens<OutT, Y, 2>(a, s);
  if (a.K <= 4) return launch_combine_tokens<OutT, Y, 4>(a, s);
  return launch_combine_tokens<OutT, Y, 8>(a, s);
}

template <typename OutT>
__global__ __launch_bounds__(kThreads) void cast_kernel(const float* src, OutT* dst, size_t n) {
  for (size_t i = blockIdx.x * static_cast<size_t>(kThreads) + threadIdx.x; i < n;
       i += static_cast<size_t>(gridDim.x) * kThreads)
    dst[i] = from_f32<OutT>(src[i]);
}

template <typename OutT, int V, int NT>
hipError_t launch_combine_v(const CombineArgs& a, int dtype, hipStream_t s) {
  const dim3 grid(a.T, (a.H + NT * V - 1) / (NT * V)), block(NT);
  if (a.y16) {
    if (a.splits != 1 || dtype == MOE355_F32) return hipErrorInvalidValue;
    if (dtype == MOE355_BF16)
      combine_kernel<OutT, bf16, 1, V, NT><<<grid, block, 0, s>>>(a);
    else
      combine_kernel<OutT, f16, 1, V, NT><<<grid, block, 0, s>>>(a);
    return hipGetLastError();
  }
  switch (a.splits) {
    case 1: combine_kernel<OutT, float, 1, V, NT><<<grid, block, 0, s>>>(a); break;
    case 2: combine_kernel<OutT, float, 2, V, NT><<<grid, block, 0, s>>>(a); break;
    case 4: combine_kernel<OutT, float, 4, V, NT><<<grid, block, 0, s>>>(a); break;
    case 8: combine_kernel<OutT, float, 8, V, NT><<<grid, block, 0, s>>>(a); break;
    case 16: combine_kernel<OutT, float, 16, V, NT><<<grid, block, 0, s>>>(a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

// Token counts whose 8-feature, 256-thread workgroups would not cover the CUs
// twice run 4 features per thread in 64-thread workgroups instead: a decode
// step's few tokens then spread over many CUs (Mixtral shape, one token: 16
// workgroups of 16 KB each rather than 2 of 128 KB). Larger counts with one
// y plane take several tokens per workgroup (combine_tokens_kernel).
template <typename OutT>
hipError_t launch_combine_t(const CombineArgs& a, int dtype, hipStream_t s) {
  const long long wide = static_cast<long long>(a.T) * ((a.H + 2047) / 2048);
  if (a.H % 8 == 0 && wide >= 2ll * device_cu_count()) {
    if (a.splits == 1 && a.K <= 8) {
      if (!a.y16) return launch_combine_tokens_k<OutT, float>(a, s);
      if (dtype == MOE355_BF16) return launch_combine_tokens_k<OutT, bf16>(a, s);
      if (dtype == MOE355_F16) return launch_combine_tokens_k<OutT, f16>(a, s);
      return hipErrorInvalidValue;
    }
    return launch_combine_v<OutT, 8, kThreads>(a, dtype, s);
  }
  return launch_combine_v<OutT, 4, kWave>(a, dtype, s);
}

// Zero-copy staging for the CPU/GPU split forward (the host buffers are
// mapped, coherent pinned memory): a kernel moves a decode step's few bytes
// between HBM and host memory itself, so nothing waits on the DMA engines,
// which the background expert copies keep busy.
__global__ __launch_bounds__(kThreads) void copy_bytes_kernel(const uint8_t* src, uint8_t* dst,
                                                             size_t n) {
  const size_t stride = static_cast<size_t>(gridDim.x) * kThreads;
  const size_t n16 = n / 16;
  const size_t t = blockIdx.x * static_cast<size_t>(kThreads) + threadIdx.x;
  for (size_t i = t; i < n16; i += stride)
    reinterpret_cast<uint4*>(dst)[i] = reinterpret_cast<const uint4*>(src)[i];
  for (size_t i = n16 * 16 + t; i < n; i += stride) dst[i] = src[i];
}

// Up to kMaxRegions regions in one launch (each grid-strided in turn): the
// routing and hidden states a split step hands to the host, so that one
// kernel, and one release of its writes to host memory, serves them all.
__global__ __launch_bounds__(kThreads) void copy_regions_kernel(const CopyRegions r) {
  const size_t stride = static_cast<size_t>(gridDim.x) * kThreads;
  const size_t t = blockIdx.x * static_cast<size_t>(kThreads) + threadIdx.x;
  for (int k = 0; k < r.count; ++k) {
    const size_t n = r.bytes[k], n16 = n / 16;
    for (size_t i = t; i < n16; i += stride)
      reinterpret_cast<uint4*>(r.dst[k])[i] = reinterpret_cast<const uint4*>(r.src[k])[i];
    for (size_t i = n16 * 16 + t; i < n; i += stride) r.dst[k][i] = r.src[k][i];
  }
}

// out = acc + host, rounded once to OutT: the host half of the split forward
// read straight from host memory (16-byte vectors; n a multiple of 4).
template <typename OutT>
__global__ __launch_bounds__(kThreads) void merge_host_kernel(const float4* acc,
                                                             const float4* host, OutT* out,
                                                             size_t n4) {
  for (size_t i = blockIdx.x * static_cast<size_t>(kThreads) + threadIdx.x; i < n4;
       i += static_cast<size_t>(gridDim.x) * kThreads) {
    const float4 a = acc[i], h = host[i];
    out[4 * i + 0] = from_f32<OutT>(a.x + h.x);
    out[4 * i + 1] = from_f32<OutT>(a.y + h.y);
    out[4 * i + 2] = from_f32<OutT>(a.z + h.z);
    out[4 * i + 3] = from_f32<OutT>(a.w + h.w);
  }
}

}  // namespace

hipError_t launch_copy_bytes(const void* src, void* dst, size_t n, hipStream_t s) {
  if (n == 0) return hipSuccess;
  size_t blocks = (n / 16 + kThreads - 1) / kThreads;
  if (blocks < 1) blocks = 1;
  if (blocks > 1024) blocks = 1024;
  copy_bytes_kernel<<<dim3(blocks), dim3(kThreads), 0, s>>>(static_cast<const uint8_t*>(src),
                                                           static_cast<uint8_t*>(dst), n);
  return hipGetLastError();
}

hipError_t launch_copy_regions(const CopyRegions& r, hipStream_t s) {
  size_t most = 0;
  for (int k = 0; k < r.count; ++k) most = r.bytes[k] > most ? r.bytes[k] : most;
  if (most == 0) return hipSuccess;
  size_t blocks = (most / 16 + kThreads - 1) / kThreads;
  if (blocks < 1) blocks = 1;
  if (blocks > 1024) blocks = 1024;
  copy_regions_kernel<<<dim3(blocks), dim3(kThreads), 0, s>>>(r);
  return hipGetLastError();
}

hipError_t launch_merge_host(const float* acc, const float* host, void* out, size_t n, int dtype,
                             hipStream_t s) {
  if (n == 0) return hipSuccess;
  const size_t n4 = n / 4;
  size_t blocks = (n4 + kThreads - 1) / kThreads;
  if (blocks > 4096) blocks = 4096;
  const float4* a = reinterpret_cast<const float4*>(acc);
  const float4* h = reinterpret_cast<const float4*>(host);
  if (dtype == MOE355_BF16)
    merge_host_kernel<bf16><<<dim3(blocks), dim3(kThreads), 0, s>>>(a, h, static_cast<bf16*>(out),
                                                                    n4);
  else if (dtype == MOE355_F16)
    merge_host_kernel<f16><<<dim3(blocks), dim3(kThreads), 0, s>>>(a, h, static_cast<f16*>(out),
                                                                   n4);
  else
    merge_host_kernel<float><<<dim3(blocks), dim3(kThreads), 0, s>>>(a, h,
                                                                     static_cast<float*>(out), n4);
  return hipGetLastError();
}

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
