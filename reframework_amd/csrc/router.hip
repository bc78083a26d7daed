// Router GEMV + softmax + top-k, one workgroup per 1-8 tokens.
//
// Replaces FusedMoE.route (reframework/moe/moe_layer.py:320-344): the router
// F.linear (:324) and torch_fused_topk (reframework/moe/fused.py:32-46). The
// router product is tiny (2*H*E flops per token) and HBM/L2 bound, so it runs
// on the VALU with fp32 accumulation; the gate matrix (E*H*2 bytes) stays in L2
// across tokens. Selection happens on the fp32 logits, which is monotone with
// the softmax the reference ranks by; exact ties go to the lower expert id.
#include <climits>

#include "common.h"
#include "dma_pipe.h"

namespace moe355 {
namespace {

constexpr int kThreads = 256;
#include "topk_wave.h"

// TB tokens per workgroup share every gate-row load (the gate matrix is read
// once per TB tokens from L2). Per thread: TB x EG partial dot products (EG
// experts per pass over the row) over its slice of H, folded across the wave
// by transpose_reduce and across the 4 waves through LDS.
template <typename T, int TB, int EG>
__global__ __launch_bounds__(kThreads) void router_kernel(const RouterArgs a) {
  constexpr int V = Vec16<T>::N;
  constexpr int NV = TB * EG;            // partial sums per thread (<= 64)
  static_assert(NV <= 64, "one value per lane after the transposed reduction");
  constexpr int SH = 6 - log2i(NV);      // lane bits below the value index
  __shared__ float part[kThreads / kWave][64];
  __shared__ float lg[TB][kMaxExperts];
  __shared__ float psel[kThreads / kWave][kMaxExperts];
  __shared__ int32_t isel[kThreads / kWave][kMaxExperts];

  const int t0 = blockIdx.x * TB;
  const int ntok = min(TB, a.T - t0);
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave;
  const int nch = a.H / V;
  const T* x = static_cast<const T*>(a.x) + static_cast<size_t>(t0) * a.H;
  const T* gate = static_cast<const T*>(a.gate);

  for (int e0 = 0; e0 < a.E; e0 += EG) {
    float acc[NV];
#pragma unroll
    for (int i = 0; i < NV; ++i) acc[i] = 0.f;
    // U chunks per thread per pass (two for one token and 8 experts, whose
    // registers allow it): every load of the pass is issued before any is used
    // (rows past the last token or expert, and chunks past the row end, are
    // clamped in bounds and their products dropped), so the U * (TB + EG)
    // loads are in flight together instead of one HBM round trip each.
    constexpr int U = TB == 1 && EG == 8 ? 2 : 1;
    for (int c0 = tid; c0 < nch; c0 += U * kThreads) {
      u32x4 xraw[U][TB], graw[U][EG];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int c = min(c0 + u * kThreads, nch - 1);
#pragma unroll
        for (int t = 0; t < TB; ++t)
          xraw[u][t] = *reinterpret_cast<const u32x4*>(x + static_cast<size_t>(min(t, ntok - 1)) * a.H + c * V);
#pragma unroll
        for (int j = 0; j < EG; ++j)
          graw[u][j] = *reinterpret_cast<const u32x4*>(gate + static_cast<size_t>(min(e0 + j, a.E - 1)) * a.H + c * V);
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        if (c0 + u * kThreads >= nch) break;
        float xf[TB][V];
#pragma unroll
        for (int t = 0; t < TB; ++t) Vec16<T>::unpack(xraw[u][t], xf[t]);
#pragma unroll
        for (int j = 0; j < EG; ++j) {
          float gf[V];
          Vec16<T>::unpack(graw[u][j], gf);
#pragma unroll
          for (int t = 0; t < TB; ++t)
#pragma unroll
            for (int q = 0; q < V; ++q) acc[t * EG + j] = fmaf(xf[t][q], gf[q], acc[t * EG + j]);
        }
      }
    }
    const float r = transpose_reduce<NV>(acc, lane);
    if ((lane & ((1 << SH) - 1)) == 0) part[wave][lane >> SH] = r;
    __syncthreads();
    for (int i = tid; i < NV; i += kThreads) {
      const int t = i / EG, e = e0 + i % EG;
      if (t < ntok && e < a.E) {
        float l = (part[0][i] + part[1][i]) + (part[2][i] + part[3][i]);
        if (a.round_logits) l = to_f32(from_f32<T>(l));
        if (a.bias) l += a.bias[e];
        lg[t][e] = l;
        if (a.logits_out) a.logits_out[static_cast<size_t>(t0 + t) * a.E + e] = l;
      }
    }
    __syncthreads();
  }

  for (int t = wave; t < ntok; t += kThreads / kWave)
    wave_topk(lg[t], a.E, a.K, a.renormalize, a.entropy_k_min, psel[wave], isel[wave],
              a.topk_w + static_cast<size_t>(t0 + t) * a.out_ld,
              a.topk_ids + static_cast<size_t>(t0 + t) * a.out_ld, lane);
}

template <typename T>
struct Mfma16R;

template <>
struct Mfma16R<bf16> {
  __device__ __forceinline__ static f32x4 mma(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
};

template <>
struct Mfma16R<f16> {
  __device__ __forceinline__ static f32x4 mma(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
};

// Prefill-sized router on MFMA: 16 tokens per workgroup, the 4 waves splitting
// H in quarters. Each wave multiplies its 16 token rows (A, 16 x 32 per step)
// by 16-expert groups of gate rows (B) with v_mfma_f32_16x16x32; the 4
// quarter sums are added in fixed order through LDS. Lane l then holds logits
// of tokens 4 (l / 16) + 0..3 for expert l % 16 of each group. A group of 16
// lanes per token does the softmax and top-k (group16_topk).
// Operands go through the LDS: a wave streams its quarter of the token and
// gate rows in batches of 64 k (128 bytes of each row) with direct-to-LDS
// loads of 8 whole rows each, up to 7 batches in flight in its own ring, and reads them
// back in MFMA layout (16-byte chunks XOR-swizzled by row, conflict free).
// Loading the MFMA layout straight from memory put the 4 lanes of a row 16
// lanes apart, so every load left as 64 separate 16-byte pieces, and the
// kernel took ~10 us at 8 experts and ~17 us at 64 whatever the token count
// (now 8.5 and 12.3 us at 4096 tokens, H = 4096 and 2048).
// The fp32 VALU router re-reads the gate per 8 tokens and spends E*H FMAs per
// token on the VALU: at 4096 tokens, 64 experts and H = 2048 it took 54 us.
template <typename T, int NG>
__global__ __launch_bounds__(kThreads) void router_mfma_kernel(const RouterArgs a) {
  constexpr int kTok = 16, EP = 16 * NG, kRows = kTok + EP;
  constexpr int kLoads = kRows / 8;  // direct-to-LDS loads per batch
  constexpr int kBuf = kRows * 128;  // bytes per batch buffer
  constexpr int kWaves = kThreads / kWave;
  // Buffers per wave: as many as 160 KB hold (a workgroup has a CU to itself
  // at these token counts), all but one in flight: ~110 KB per CU, what a
  // CU needs at ~1.5 us of load latency.
  constexpr int kNB = NG == 1 ? 8 : NG == 2 ? 6 : 4;
  static_assert(kWaves * kNB * kBuf <= 160 * 1024, "LDS");
  static_assert((kNB - 1) * kLoads < 64, "vmcnt range");
  __shared__ __attribute__((aligned(1024))) uint8_t stage[kWaves][kNB][kBuf];
  // After the K loop the ring holds the quarter sums and the logits.
  typedef float Part[kWaves][kTok][EP];
  typedef float Lg[kTok][EP];
  static_assert(sizeof(Part) + sizeof(Lg) <= sizeof(stage), "LDS reuse");
  Part& part = *reinterpret_cast<Part*>(&stage[0][0][0]);
  Lg& lg = *reinterpret_cast<Lg*>(&stage[0][0][0] + sizeof(Part));
  const int t0 = blockIdx.x * kTok;
  const int tid = threadIdx.x, lane = tid & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int r = lane & 15, kq = lane >> 4;
  const int hq = a.H / kWaves;
  const uint32_t pitch = static_cast<uint32_t>(a.H) * sizeof(T);
  // Load q covers batch rows 8 q .. 8 q + 7 (rows 0-15 tokens t0.., then gate
  // rows): lane l takes row 8 q + l / 8 and lands in its LDS chunk l % 8,
  // which holds logical chunk (l % 8) ^ ((row >> 1) & 7). Token rows past T
  // and gate rows past E load the last row again (never read back).
  const __amdgpu_buffer_rsrc_t xsrc =
      pipe::lds_rsrc(static_cast<const T*>(a.x) + static_cast<size_t>(t0) * a.H + wave * hq);
  const __amdgpu_buffer_rsrc_t gsrc = pipe::lds_rsrc(static_cast<const T*>(a.gate) + wave * hq);
  uint32_t voff[kLoads];
#pragma unroll
  for (int q = 0; q < kLoads; ++q) {
    const int row = 8 * q + (lane >> 3), c = (lane & 7) ^ ((row >> 1) & 7);
    const int src = row < kTok ? min(t0 + row, a.T - 1) - t0 : min(row - kTok, a.E - 1);
    voff[q] = static_cast<uint32_t>(src) * pitch + c * 16;
  }
  auto issue = [&](int b) {
    uint8_t* dst = &stage[wave][b % kNB][0];
#pragma unroll
    for (int q = 0; q < kLoads; ++q)
      pipe::dma16_rsrc(q < kTok / 8 ? xsrc : gsrc, voff[q], b * 128, dst + q * 1024);
  };
  // Fragment of batch row `row`, step u (32 k) of the batch: lane (r, kq) reads
  // logical chunk 4 u + kq.
  auto frag = [&](const uint8_t* buf, int row, int u) {
    return *reinterpret_cast<const u32x4*>(buf + row * 128 + (((4 * u + kq) ^ ((row >> 1) & 7)) << 4));
  };
  f32x4 acc[NG];
#pragma unroll
  for (int g = 0; g < NG; ++g) acc[g] = f32x4{0.f, 0.f, 0.f, 0.f};
  const int nb = hq / 64;
  for (int b = 0; b < kNB - 1 && b < nb; ++b) issue(b);
  for (int b = 0; b < nb; ++b) {
    // The buffer of batch b + kNB - 1 held batch b - 1, whose reads have
    // completed. Then wait until only the batches after b are in flight.
    if (b + kNB - 1 < nb) issue(b + kNB - 1);
    switch (min(nb - 1 - b, kNB - 1)) {
      case 0: pipe::wait_vmcnt<0>(); break;
      case 1: pipe::wait_vmcnt<kLoads>(); break;
      case 2: pipe::wait_vmcnt<2 * kLoads>(); break;
      case 3: pipe::wait_vmcnt<3 * kLoads>(); break;
      case 4: pipe::wait_vmcnt<4 * kLoads>(); break;
      case 5: pipe::wait_vmcnt<(kNB > 5 ? 5 : 1) * kLoads>(); break;
      case 6: pipe::wait_vmcnt<(kNB > 6 ? 6 : 1) * kLoads>(); break;
      default: pipe::wait_vmcnt<(kNB > 7 ? 7 : 1) * kLoads>(); break;
    }
    const uint8_t* buf = &stage[wave][b % kNB][0];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const u32x4 av = frag(buf, r, u);
#pragma unroll
      for (int g = 0; g < NG; ++g) acc[g] = Mfma16R<T>::mma(av, frag(buf, kTok + 16 * g + r, u), acc[g]);
    }
    pipe::wait_lgkm0();
  }
  __syncthreads();
#pragma unroll
  for (int g = 0; g < NG; ++g)
#pragma unroll
    for (int i = 0; i < 4; ++i) part[wave][4 * kq + i][16 * g + r] = acc[g][i];
  __syncthreads();
  for (int i = tid; i < kTok * EP; i += kThreads) {
    const int t = i / EP, e = i % EP;
    if (t0 + t < a.T && e < a.E) {
      float l = (part[0][t][e] + part[1][t][e]) + (part[2][t][e] + part[3][t][e]);
      if (a.round_logits) l = to_f32(from_f32<T>(l));
      if (a.bias) l += a.bias[e];
      lg[t][e] = l;
      if (a.logits_out) a.logits_out[static_cast<size_t>(t0 + t) * a.E + e] = l;
    }
  }
  __syncthreads();
  // 16 lanes per token (tid = 16 t + sub).
  const int tt = tid / 16;
  if (t0 + tt < a.T)
    group16_topk<NG>(lg[tt], a.E, a.K, a.renormalize, a.entropy_k_min,
                     a.topk_w + static_cast<size_t>(t0 + tt) * a.out_ld,
                     a.topk_ids + static_cast<size_t>(t0 + tt) * a.out_ld, tid & 15);
}

// Router logits only, for a few tokens over many experts: one workgroup per
// (token, EG experts). The one-workgroup-per-token kernel pulls the whole gate
// (E*H*2 bytes) through one CU per token, and a CU's load bandwidth bounds it
// (64 experts, H = 2048, 8 tokens: 15.7 us for 256 KB per workgroup); here the
// gate is spread over T*E/EG workgroups. The logits (rounded, plus the bias)
// go to logits_out, and topk_logits_kernel selects from them.
template <typename T, int EG>
__global__ __launch_bounds__(kThreads) void router_logits_kernel(const RouterArgs a) {
  constexpr int V = Vec16<T>::N;
  constexpr int SH = 6 - log2i(EG);
  constexpr int U = 2;  // chunks per thread per iteration, all loads issued first
  __shared__ float part[kThreads / kWave][64];
  const int t = blockIdx.x, e0 = blockIdx.y * EG;
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave;
  const int nch = a.H / V;
  const T* x = static_cast<const T*>(a.x) + static_cast<size_t>(t) * a.H;
  const T* gate = static_cast<const T*>(a.gate);
  float acc[EG];
#pragma unroll
  for (int j = 0; j < EG; ++j) acc[j] = 0.f;
  for (int c0 = tid; c0 < nch; c0 += U * kThreads) {
    u32x4 xraw[U], graw[U][EG];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = min(c0 + u * kThreads, nch - 1);
      xraw[u] = *reinterpret_cast<const u32x4*>(x + c * V);
#pragma unroll
      for (int j = 0; j < EG; ++j)
        graw[u][j] = *reinterpret_cast<const u32x4*>(
            gate + static_cast<size_t>(min(e0 + j, a.E - 1)) * a.H + c * V);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (c0 + u * kThreads >= nch) break;
      float xf[V];
      Vec16<T>::unpack(xraw[u], xf);
#pragma unroll
      for (int j = 0; j < EG; ++j) {
        float gf[V];
        Vec16<T>::unpack(graw[u][j], gf);
#pragma unroll
        for (int q = 0; q < V; ++q) acc[j] = fmaf(xf[q], gf[q], acc[j]);
      }
    }
  }
  const float r = transpose_reduce<EG>(acc, lane);
  if ((lane & ((1 << SH) - 1)) == 0) part[wave][lane >> SH] = r;
  __syncthreads();
  if (tid < EG && e0 + tid < a.E) {
    float l = (part[0][tid] + part[1][tid]) + (part[2][tid] + part[3][tid]);
    if (a.round_logits) l = to_f32(from_f32<T>(l));
    if (a.bias) l += a.bias[e0 + tid];
    a.logits_out[static_cast<size_t>(t) * a.E + e0 + tid] = l;
  }
}

// One wave per token on given fp32 logits (logits_in, or the logits_out the
// split router just wrote); results at row t of [T, out_ld] arrays.
__global__ __launch_bounds__(kThreads) void topk_logits_kernel(const RouterArgs a) {
  __shared__ float psel[kThreads / kWave][kMaxExperts];
  __shared__ int32_t isel[kThreads / kWave][kMaxExperts];
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
  const int t = blockIdx.x * (kThreads / kWave) + wave;
  if (t >= a.T) return;
  wave_topk(a.logits_in + static_cast<size_t>(t) * a.E, a.E, a.K, a.renormalize,
            a.entropy_k_min, psel[wave], isel[wave],
            a.topk_w + static_cast<size_t>(t) * a.out_ld,
            a.topk_ids + static_cast<size_t>(t) * a.out_ld, lane);
}

}  // namespace

template <typename T>
hipError_t launch_router_t(const RouterArgs& a, hipStream_t s) {
  // Experts per pass over the row: as many as the 64 per-thread sums allow
  // for the workgroup's token count, so E = 64 at one token costs two passes
  // (two memory round trips) rather than eight.
  const dim3 block(kThreads);
  if constexpr (!std::is_same<T, float>::value) {
    // Prefill sizes on MFMA (16 tokens per workgroup); the VALU kernels keep
    // the smaller sizes, where one workgroup per 1-8 tokens has the lowest
    // latency (256-768 tokens: 7.8 against 9.5 us at 8 experts; at 64
    // experts MFMA wins from 256 tokens, 17 against 23 us).
    if ((a.T >= 1024 || (a.T >= 256 && a.E > 16)) && a.K <= 8 && a.E <= 64 && a.H % 256 == 0) {
      const dim3 grid((a.T + 15) / 16);
      if (a.E <= 16)
        router_mfma_kernel<T, 1><<<grid, block, 0, s>>>(a);
      else if (a.E <= 32)
        router_mfma_kernel<T, 2><<<grid, block, 0, s>>>(a);
      else
        router_mfma_kernel<T, 4><<<grid, block, 0, s>>>(a);
      return hipGetLastError();
    }
  }
  if (a.logits_out && a.T < 256 && a.E > 16) {
    // Few tokens over many experts, with a logits buffer to pass through: the
    // logits over (token, 8 experts) workgroups, then the selection (64
    // experts, H = 2048, 8 tokens: 15.7 -> ~6 us).
    router_logits_kernel<T, 8><<<dim3(a.T, (a.E + 7) / 8), block, 0, s>>>(a);
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) return err;
    RouterArgs b = a;
    b.logits_in = a.logits_out;
    const int per = kThreads / kWave;
    topk_logits_kernel<<<dim3((a.T + per - 1) / per), block, 0, s>>>(b);
    return hipGetLastError();
  }
  if (a.T >= 1024)
    router_kernel<T, 8, 8><<<dim3((a.T + 7) / 8), block, 0, s>>>(a);
  else if (a.T >= 256 && a.E > 8)
    router_kernel<T, 4, 16><<<dim3((a.T + 3) / 4), block, 0, s>>>(a);
  else if (a.T >= 256)
    router_kernel<T, 4, 8><<<dim3((a.T + 3) / 4), block, 0, s>>>(a);
  else if (a.E > 16)
    router_kernel<T, 1, 32><<<dim3(a.T), block, 0, s>>>(a);
  else if (a.E > 8)
    router_kernel<T, 1, 16><<<dim3(a.T), block, 0, s>>>(a);
  else
    router_kernel<T, 1, 8><<<dim3(a.T), block, 0, s>>>(a);
  return hipGetLastError();
}

hipError_t launch_router(const RouterArgs& a, int dtype, hipStream_t s) {
  if (a.T == 0) return hipSuccess;
  if (dtype == MOE355_BF16) return launch_router_t<bf16>(a, s);
  if (dtype == MOE355_F16) return launch_router_t<f16>(a, s);
  return launch_router_t<float>(a, s);
}

hipError_t launch_topk_from_logits(const RouterArgs& a, hipStream_t s) {
  if (a.T == 0) return hipSuccess;
  const int per = kThreads / kWave;
  topk_logits_kernel<<<dim3((a.T + per - 1) / per), dim3(kThreads), 0, s>>>(a);
  return hipGetLastError();
}

}  // namespace moe355
