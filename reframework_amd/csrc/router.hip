// Router GEMV + softmax + top-k, one workgroup per token.
//
// Replaces FusedMoE.route (reframework/moe/moe_layer.py:320-344): the router
// F.linear (:324) and torch_fused_topk (reframework/moe/fused.py:32-46). The
// router product is tiny (2*H*E flops per token) and HBM/L2 bound, so it runs
// on the VALU with fp32 accumulation; the gate matrix (E*H*2 bytes) stays in L2
// across tokens. Selection happens on the fp32 logits, which is monotone with
// the softmax the reference ranks by; exact ties go to the lower expert id.
#include <climits>

#include "common.h"

namespace moe355 {
namespace {

constexpr int kThreads = 256;
constexpr int kExpGroup = 8;   // experts accumulated per pass over the row
constexpr int kMaxChunks = 8;  // 16-byte chunks of x kept in registers per thread
constexpr int kMaxPerLane = kMaxExperts / kWave;

// Softmax + top-k + renormalisation of one token's logits by one wave.
// lg: E fp32 logits (LDS or global). psel/isel: per-wave LDS scratch of E
// entries. Mirrors torch_fused_topk (fused.py:42-45) and, when kmin > 0, the
// entropy-adaptive branch of FusedMoE.route (moe_layer.py:326-342).
__device__ void wave_topk(const float* lg, int E, int K, int renorm, int kmin, float* psel,
                          int32_t* isel, float* w_out, int32_t* id_out, int lane) {
  float v[kMaxPerLane];
  bool live[kMaxPerLane];
#pragma unroll
  for (int j = 0; j < kMaxPerLane; ++j) {
    const int e = lane + kWave * j;
    live[j] = e < E;
    v[j] = live[j] ? lg[e] : -INFINITY;
  }
  float m = -INFINITY;
#pragma unroll
  for (int j = 0; j < kMaxPerLane; ++j)
    if (live[j]) m = fmaxf(m, v[j]);
  m = wave_max(m);
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < kMaxPerLane; ++j)
    if (live[j]) s += expf(v[j] - m);
  s = wave_sum(s);

  // Shannon entropy of the softmax, only for the entropy-adaptive branch.
  float hs = 0.f;
  if (kmin > 0) {
#pragma unroll
    for (int j = 0; j < kMaxPerLane; ++j) {
      if (live[j]) {
        const float p = expf(v[j] - m) / s;
        hs += p * logf(fmaxf(p, 1e-9f));
      }
    }
    hs = -wave_sum(hs);
  }

  for (int k = 0; k < K; ++k) {
    float bv = -INFINITY;
    int bi = INT_MAX;
#pragma unroll
    for (int j = 0; j < kMaxPerLane; ++j) {
      const int e = lane + kWave * j;
      if (live[j] && (v[j] > bv || (v[j] == bv && e < bi))) {
        bv = v[j];
        bi = e;
      }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      const float ov = __shfl_xor(bv, o, kWave);
      const int oi = __shfl_xor(bi, o, kWave);
      if (ov > bv || (ov == bv && oi < bi)) {
        bv = ov;
        bi = oi;
      }
    }
#pragma unroll
    for (int j = 0; j < kMaxPerLane; ++j)
      if (lane + kWave * j == bi) live[j] = false;
    if (lane == 0) {
      psel[k] = expf(bv - m) / s;
      isel[k] = bi;
    }
  }

  if (lane == 0) {
    int kd = K;
    if (kmin > 0) {
      const float hn = E > 1 ? hs / logf(static_cast<float>(E)) : 0.f;
      const float kf = rintf(static_cast<float>(kmin) + static_cast<float>(K - kmin) * hn);
      kd = static_cast<int>(fminf(fmaxf(kf, static_cast<float>(kmin)), static_cast<float>(K)));
    }
    float sum = 0.f;
    for (int k = 0; k < K; ++k) {
      const float w = k < kd ? psel[k] : 0.f;
      psel[k] = w;
      sum += w;
    }
    const bool norm = kmin > 0 || renorm;
    const float denom = kmin > 0 ? fmaxf(sum, 1e-9f) : sum;
    for (int k = 0; k < K; ++k) {
      w_out[k] = norm ? psel[k] / denom : psel[k];
      id_out[k] = isel[k];
    }
  }
}

template <typename T>
__global__ __launch_bounds__(kThreads) void router_kernel(const RouterArgs a) {
  __shared__ float part[kThreads / kWave][kMaxExperts];
  __shared__ float lg[kMaxExperts];
  __shared__ float psel[kMaxExperts];
  __shared__ int32_t isel[kMaxExperts];

  constexpr int V = Vec16<T>::N;
  const int t = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave;
  const int nch = a.H / V;
  const T* xr = static_cast<const T*>(a.x) + static_cast<size_t>(t) * a.H;
  const T* gate = static_cast<const T*>(a.gate);

  u32x4 xraw[kMaxChunks];
#pragma unroll
  for (int i = 0; i < kMaxChunks; ++i) {
    const int c = tid + kThreads * i;
    xraw[i] = c < nch ? *reinterpret_cast<const u32x4*>(xr + c * V) : u32x4{0, 0, 0, 0};
  }

  for (int e0 = 0; e0 < a.E; e0 += kExpGroup) {
    float acc[kExpGroup];
#pragma unroll
    for (int j = 0; j < kExpGroup; ++j) acc[j] = 0.f;
#pragma unroll
    for (int i = 0; i < kMaxChunks; ++i) {
      const int c = tid + kThreads * i;
      if (c < nch) {
        float xf[V];
        Vec16<T>::unpack(xraw[i], xf);
#pragma unroll
        for (int j = 0; j < kExpGroup; ++j) {
          const int e = e0 + j;
          if (e < a.E) {
            const u32x4 g =
                *reinterpret_cast<const u32x4*>(gate + static_cast<size_t>(e) * a.H + c * V);
            float gf[V];
            Vec16<T>::unpack(g, gf);
#pragma unroll
            for (int q = 0; q < V; ++q) acc[j] = fmaf(xf[q], gf[q], acc[j]);
          }
        }
      }
    }
#pragma unroll
    for (int j = 0; j < kExpGroup; ++j) {
      const float r = wave_sum(acc[j]);
      if (lane == 0 && e0 + j < a.E) part[wave][e0 + j] = r;
    }
  }
  __syncthreads();

  for (int e = tid; e < a.E; e += kThreads) {
    float l = (part[0][e] + part[1][e]) + (part[2][e] + part[3][e]);
    if (a.round_logits) l = to_f32(from_f32<T>(l));
    if (a.bias) l += a.bias[e];
    lg[e] = l;
    if (a.logits_out) a.logits_out[static_cast<size_t>(t) * a.E + e] = l;
  }
  __syncthreads();

  if (wave == 0)
    wave_topk(lg, a.E, a.K, a.renormalize, a.entropy_k_min, psel, isel,
              a.topk_w + static_cast<size_t>(t) * a.K, a.topk_ids + static_cast<size_t>(t) * a.K,
              lane);
}

// One wave per token on given fp32 logits.
__global__ __launch_bounds__(kThreads) void topk_logits_kernel(const RouterArgs a) {
  __shared__ float psel[kThreads / kWave][kMaxExperts];
  __shared__ int32_t isel[kThreads / kWave][kMaxExperts];
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
  const int t = blockIdx.x * (kThreads / kWave) + wave;
  if (t >= a.T) return;
  wave_topk(a.logits_in + static_cast<size_t>(t) * a.E, a.E, a.K, a.renormalize, 0, psel[wave],
            isel[wave], a.topk_w + static_cast<size_t>(t) * a.K,
            a.topk_ids + static_cast<size_t>(t) * a.K, lane);
}

}  // namespace

hipError_t launch_router(const RouterArgs& a, int dtype, hipStream_t s) {
  if (a.T == 0) return hipSuccess;
  const dim3 grid(a.T), block(kThreads);
  if (dtype == MOE355_BF16)
    router_kernel<bf16><<<grid, block, 0, s>>>(a);
  else if (dtype == MOE355_F16)
    router_kernel<f16><<<grid, block, 0, s>>>(a);
  else
    router_kernel<float><<<grid, block, 0, s>>>(a);
  return hipGetLastError();
}

hipError_t launch_topk_from_logits(const RouterArgs& a, hipStream_t s) {
  if (a.T == 0) return hipSuccess;
  const int per = kThreads / kWave;
  topk_logits_kernel<<<dim3((a.T + per - 1) / per), dim3(kThreads), 0, s>>>(a);
  return hipGetLastError();
}

}  // namespace moe355
