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
#include <climits>

#include "common.h"
#include "dma_pipe.h"

namespace moe355 {
namespace {

constexpr int kThreads = 256;
#include "topk_wave.h"
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

// Residual add + RMSNorm + router on TB rows per workgroup, 16-bit storage
// types: the decoder step before the MoE (reframework/models/base.py:135-136)
// in one launch. The norm is add_rmsnorm_kernel's arithmetic with the same
// per-thread chunks and reduction order, so residual_out and normed are bit
// for bit that kernel's. The normed rows then stay in registers, rounded to T
// as the reference stores them, for the router's dot products with the gate:
// fp32 sums over this thread's chunks for EG experts at a time, the gate read
// from L2 once per TB rows; folded across the wave by transpose_reduce and
// across the 4 waves through LDS; logits rounded to T (round_logits) plus the
// bias; then softmax / top-k / renormalisation by wave_topk as the router
// does (FusedMoE.route, reframework/moe/moe_layer.py:320-344). Rows past T
// load the last row again and are not stored.
//
// The kernel is a chain of dependent steps per workgroup, so every load that
// does not depend on an earlier result is issued first: the rows, the norm
// weight and bias, and (where it fits in registers, PF) the gate chunks of
// the first EG experts; each later pass's gate chunks are loaded while the
// pass before it multiplies. One memory round trip then precedes the
// arithmetic.
template <typename T, typename W, int CPT, int TB, int EG>
__global__ __launch_bounds__(kThreads) void add_rmsnorm_router_kernel(const NormArgs a,
                                                                      const RouterArgs ra) {
  constexpr int N = Vec16<T>::N;  // elements per 16-byte chunk
  constexpr int NV = TB * EG;     // router partial sums per thread
  static_assert(NV <= 64, "one value per lane after the transposed reduction");
  constexpr int SH = 6 - log2i(NV);
  constexpr int kWaves = kThreads / kWave;
  constexpr bool PF = CPT * EG <= 16;  // gate passes double-buffered (2 x 64 VGPRs at most)
  const int t0 = blockIdx.x * TB, ntok = min(TB, a.T - t0);
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave;
  const int chunks = a.H / N;
  const T* gate = static_cast<const T*>(ra.gate);
  __shared__ float red[TB][kWaves];
  __shared__ float part[kWaves][64];
  __shared__ float lg[TB][kMaxRouterExperts];
  __shared__ float psel[kWaves][kMaxRouterExperts];
  __shared__ int32_t isel[kWaves][kMaxRouterExperts];

  u32x4 npk[TB][CPT];  // the rows: residual sums, then normed, rounded to T
  u32x4 gcur[PF ? CPT : 1][PF ? EG : 1];  // this pass's gate chunks
  ParamChunk<W, N> wc[CPT], bc[CPT];
  {
    u32x4 rraw[TB][CPT];
#pragma unroll
    for (int t = 0; t < TB; ++t) {
      const size_t row = static_cast<size_t>(t0 + min(t, ntok - 1)) * a.H;
#pragma unroll
      for (int c = 0; c < CPT; ++c) {
        const int ch = tid + c * kThreads;
        if (ch < chunks) {
          npk[t][c] = *reinterpret_cast<const u32x4*>(static_cast<const T*>(a.x) + row +
                                                      static_cast<size_t>(ch) * N);
          if (a.residual)
            rraw[t][c] = *reinterpret_cast<const u32x4*>(static_cast<const T*>(a.residual) +
                                                         row + static_cast<size_t>(ch) * N);
        }
      }
    }
#pragma unroll
    for (int c = 0; c < CPT; ++c) {
      const int ch = tid + c * kThreads;
      if (ch < chunks) {
        wc[c].load(static_cast<const W*>(a.weight), ch * N);
        if (a.bias) bc[c].load(static_cast<const W*>(a.bias), ch * N);
        if constexpr (PF) {
#pragma unroll
          for (int j = 0; j < EG; ++j)
            gcur[c][j] = *reinterpret_cast<const u32x4*>(
                gate + static_cast<size_t>(min(j, ra.E - 1)) * a.H + static_cast<size_t>(ch) * N);
        }
      }
    }
#pragma unroll
    for (int t = 0; t < TB; ++t) {
      float ss = 0.f;
      const size_t row = static_cast<size_t>(t0 + t) * a.H;
#pragma unroll
      for (int c = 0; c < CPT; ++c) {
        const int ch = tid + c * kThreads;
        if (ch >= chunks) continue;
        float r[N];
        Vec16<T>::unpack(npk[t][c], r);
        if (a.residual) {
          float sv[N];
          Vec16<T>::unpack(rraw[t][c], sv);
#pragma unroll
          for (int i = 0; i < N; ++i) r[i] = to_f32(from_f32<T>(r[i] + sv[i]));
          npk[t][c] = pack16<T>(r);
          if (t < ntok)
            *reinterpret_cast<u32x4*>(static_cast<T*>(a.residual_out) + row +
                                      static_cast<size_t>(ch) * N) = npk[t][c];
        }
#pragma unroll
        for (int i = 0; i < N; ++i) ss += r[i] * r[i];
      }
      ss = wave_sum(ss);
      if (lane == 0) red[t][wave] = ss;
    }
  }
  __syncthreads();
#pragma unroll
  for (int t = 0; t < TB; ++t) {
    float tot = 0.f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) tot += red[t][w];
    const float inv = 1.0f / sqrtf(tot / static_cast<float>(a.H) + a.eps);
    const size_t row = static_cast<size_t>(t0 + t) * a.H;
#pragma unroll
    for (int c = 0; c < CPT; ++c) {
      const int ch = tid + c * kThreads;
      if (ch >= chunks) continue;
      float r[N], wv[N], bv[N], o[N];
      Vec16<T>::unpack(npk[t][c], r);
      wc[c].unpack(wv);
      if (a.bias) bc[c].unpack(bv);
#pragma unroll
      for (int i = 0; i < N; ++i) {
        o[i] = r[i] * inv * wv[i];
        if (a.bias) o[i] += bv[i];
      }
      npk[t][c] = pack16<T>(o);
      if (t < ntok)
        *reinterpret_cast<u32x4*>(static_cast<T*>(a.out) + row + static_cast<size_t>(ch) * N) =
            npk[t][c];
    }
  }

  // One pass per EG experts: the logits of experts e0 .. e0+EG-1 for the TB rows.
  for (int e0 = 0; e0 < ra.E; e0 += EG) {
    const bool more = e0 + EG < ra.E;
    u32x4 gnext[PF ? CPT : 1][PF ? EG : 1];
    if constexpr (PF) {
      if (more) {
#pragma unroll
        for (int c = 0; c < CPT; ++c) {
          const int ch = tid + c * kThreads;
          if (ch < chunks) {
#pragma unroll
            for (int j = 0; j < EG; ++j)
              gnext[c][j] = *reinterpret_cast<const u32x4*>(
                  gate + static_cast<size_t>(min(e0 + EG + j, ra.E - 1)) * a.H +
                  static_cast<size_t>(ch) * N);
          }
        }
      }
    }
    float acc[NV];
#pragma unroll
    for (int i = 0; i < NV; ++i) acc[i] = 0.f;
#pragma unroll
    for (int c = 0; c < CPT; ++c) {
      const int ch = tid + c * kThreads;
      if (ch >= chunks) continue;
      u32x4 graw[EG];
#pragma unroll
      for (int j = 0; j < EG; ++j) {
        if constexpr (PF)
          graw[j] = gcur[c][j];
        else
          graw[j] = *reinterpret_cast<const u32x4*>(
              gate + static_cast<size_t>(min(e0 + j, ra.E - 1)) * a.H + static_cast<size_t>(ch) * N);
      }
      float xf[TB][N];
#pragma unroll
      for (int t = 0; t < TB; ++t) Vec16<T>::unpack(npk[t][c], xf[t]);
#pragma unroll
      for (int j = 0; j < EG; ++j) {
        float gf[N];
        Vec16<T>::unpack(graw[j], gf);
#pragma unroll
        for (int t = 0; t < TB; ++t)
#pragma unroll
          for (int q = 0; q < N; ++q) acc[t * EG + j] = fmaf(xf[t][q], gf[q], acc[t * EG + j]);
      }
    }
    const float r = transpose_reduce<NV>(acc, lane);
    if ((lane & ((1 << SH) - 1)) == 0) part[wave][lane >> SH] = r;
    __syncthreads();
    for (int i = tid; i < NV; i += kThreads) {
      const int t = i / EG, e = e0 + i % EG;
      if (t < ntok && e < ra.E) {
        float l = (part[0][i] + part[1][i]) + (part[2][i] + part[3][i]);
        if (ra.round_logits) l = to_f32(from_f32<T>(l));
        if (ra.bias) l += ra.bias[e];
        lg[t][e] = l;
        if (ra.logits_out) ra.logits_out[static_cast<size_t>(t0 + t) * ra.E + e] = l;
      }
    }
    __syncthreads();
    if constexpr (PF) {
      if (more) {
#pragma unroll
        for (int c = 0; c < CPT; ++c)
#pragma unroll
          for (int j = 0; j < EG; ++j) gcur[c][j] = gnext[c][j];
      }
    }
  }
  for (int t = wave; t < ntok; t += kWaves)
    wave_topk(lg[t], ra.E, ra.K, ra.renormalize, 0, psel[wave], isel[wave],
              ra.topk_w + static_cast<size_t>(t0 + t) * ra.out_ld,
              ra.topk_ids + static_cast<size_t>(t0 + t) * ra.out_ld, lane);
}

// Workgroup barrier after this wave's LDS accesses have completed; unlike
// __syncthreads it does not wait for the wave's global loads and stores.
__device__ __forceinline__ void lds_barrier() {
  pipe::wait_lgkm0();
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_barrier();
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

constexpr int kNormRouterRows = 8;  // rows per workgroup of the prefill kernel

// Residual add + RMSNorm + router at prefill sizes, 8 rows per workgroup, up
// to 16 experts, H a multiple of 256 up to 2048 * CPT. The two-kernel path
// there (add_rmsnorm_kernel, then the router's router_mfma_kernel) writes the
// normed rows to HBM and reads them back; here they stay in an LDS tile:
//   1. every load is issued at once: x rows straight into the tile with
//      direct-to-LDS loads, residual rows into registers. After one wait,
//      x + residual rounded to T goes back into the tile, and each thread sums
//      its squares per row;
//   2. the gate fragments of phase 3 are loaded (before any store, so that
//      waiting for them does not wait for the stores); then per row the scale
//      from the wave sums, and the thread's chunks of the tile go to
//      residual_out, are scaled by it and the weight (+ bias), rounded to T,
//      and go to out and back into the tile. Chunks, sums and their order are
//      add_rmsnorm_kernel's, so residual_out and out are bit for bit its;
//   3. the router's product with the same MFMA sequence per wave as
//      router_mfma_kernel for one 16-expert group (wave w over the quarter
//      [w H/4, (w+1) H/4), 32 k a step, ascending), A fragments from the tile
//      (fragment rows 8-15 repeat rows 0-7; their results are dropped) and B
//      fragments of the gate in registers (the gate is L2 resident); the
//      quarter sums, the rounded logits plus bias and group16_topk follow
//      that kernel, so logits and routing are bit for bit the two-kernel
//      path's.
// Eight rows (a 64 KB tile at H = 4096) let two workgroups share a CU. With
// sixteen a workgroup had its CU to itself, its reads and its writes never
// overlapped, and the kernel lost to the two-kernel path (4096 rows, H = 4096,
// 8 experts: 36 against 31 us; with eight rows 28 us, and 54 against 58 us at
// 8192 rows).
// The tile holds row t's 16-byte chunk c at slot c ^ t of its row (rows
// 2048 * CPT elements apart): the lanes of an MFMA fragment read its rows at
// one chunk from distinct slots of one 128-byte span (conflict free). The
// lane of thread tid fills slot tid + 256 c of each row, so the chunk a
// thread works on in phases 1 and 2 (slot (tid + 256 c) ^ t) was loaded by
// lane tid ^ t of its own wave: waiting for the wave's own loads suffices.
// Slots past the row end (rows are the largest H apart) load zeros without
// touching memory. Rows past T load the last row again and are not stored;
// their logits are not written. Barriers wait for LDS only (s_waitcnt
// lgkmcnt(0) + s_barrier): __syncthreads would also wait for the global
// stores and the gate loads in flight.
template <typename T, typename W, int CPT>
__global__ __launch_bounds__(kThreads) void add_rmsnorm_router_mfma_kernel(const NormArgs a,
                                                                           const RouterArgs ra) {
  constexpr int N = Vec16<T>::N;  // elements per 16-byte chunk
  constexpr int kTok = kNormRouterRows, kWaves = kThreads / kWave;
  constexpr int kMaxH = CPT * kThreads * N;
  constexpr int kPitch = kMaxH * static_cast<int>(sizeof(T));  // tile row, bytes
  constexpr int kMaxB = kMaxH / 256;      // 64-k batches of a wave's quarter
  __shared__ __attribute__((aligned(1024))) uint8_t tile[kTok * kPitch];
  __shared__ float red[kTok][kWaves];
  __shared__ float part[kWaves][16][16];
  __shared__ float lg[kTok][16];
  static_assert(sizeof(tile) + sizeof(red) + sizeof(part) + sizeof(lg) <= 160 * 1024, "LDS");

  const int t0 = blockIdx.x * kTok, ntok = min(kTok, a.T - t0);
  const int tid = threadIdx.x, lane = tid & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int chunks = a.H / N;
  const uint32_t rowbytes = static_cast<uint32_t>(a.H) * sizeof(T);
  const bool has_res = a.residual != nullptr;
  auto slot = [&](int t, int ch) -> u32x4* {
    return reinterpret_cast<u32x4*>(tile + t * kPitch + ((ch ^ t) << 4));
  };

  ParamChunk<W, N> wc[CPT], bc[CPT];
#pragma unroll
  for (int c = 0; c < CPT; ++c) {
    const int ch = tid + c * kThreads;
    if (ch < chunks) {
      wc[c].load(static_cast<const W*>(a.weight), ch * N);
      if (a.bias) bc[c].load(static_cast<const W*>(a.bias), ch * N);
    }
  }
  float ss[kTok];
  {
    const __amdgpu_buffer_rsrc_t xsrc =
        pipe::lds_rsrc(static_cast<const T*>(a.x) + static_cast<size_t>(t0) * a.H);
    u32x4 rs[kTok][CPT];
#pragma unroll
    for (int t = 0; t < kTok; ++t) {
      const int src = min(t, ntok - 1);
#pragma unroll
      for (int c = 0; c < CPT; ++c) {
        const int s = tid + c * kThreads;  // the slot this lane fills, holding chunk s ^ t
        const uint32_t off = s < chunks ? static_cast<uint32_t>(src) * rowbytes +
                                              (static_cast<uint32_t>(s ^ t) << 4)
                                        : pipe::kPadOffset;
        pipe::dma16_rsrc(xsrc, off, 0, tile + t * kPitch + (wave * kWave + c * kThreads) * 16);
        if (has_res && s < chunks)
          rs[t][c] = *reinterpret_cast<const u32x4*>(
              static_cast<const T*>(a.residual) + static_cast<size_t>(t0 + src) * a.H +
              static_cast<size_t>(s) * N);
      }
    }
    // All loads at once (a CU holds its 16 rows in flight), then one wait on
    // every path: later LDS reads need no wait for the direct-to-LDS loads.
    pipe::wait_vmcnt<0>();
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
#pragma unroll
    for (int t = 0; t < kTok; ++t) {
      ss[t] = 0.f;
#pragma unroll
      for (int c = 0; c < CPT; ++c) {
        const int ch = tid + c * kThreads;
        if (ch >= chunks) continue;
        u32x4* p = slot(t, ch);
        float v[N];
        Vec16<T>::unpack(*p, v);
        if (has_res) {
          float sv[N];
          Vec16<T>::unpack(rs[t][c], sv);
          // the sum is rounded to the storage dtype, as the reference adds there
#pragma unroll
          for (int i = 0; i < N; ++i) v[i] = to_f32(from_f32<T>(v[i] + sv[i]));
          *p = pack16<T>(v);
        }
#pragma unroll
        for (int i = 0; i < N; ++i) ss[t] += v[i] * v[i];
      }
    }
  }
#pragma unroll
  for (int t = 0; t < kTok; ++t) {
    const float s = wave_sum(ss[t]);
    if (lane == 0) red[t][wave] = s;
  }

  // The gate's B fragments for phase 3, loaded before any store so that
  // waiting for them does not wait for the stores: lane (r, kq) of wave w
  // holds gate row min(r, E - 1), elements w H/4 + 64 b + 32 u + 8 kq .. + 7
  // (rows past E load the last row again; their columns are dropped).
  const int r16 = lane & 15, kq = lane >> 4;
  const int nb = a.H / 256;
  u32x4 gf[kMaxB][2];
  {
    const T* grow = static_cast<const T*>(ra.gate) + static_cast<size_t>(min(r16, ra.E - 1)) * a.H +
                    wave * (a.H / kWaves) + kq * 8;
#pragma unroll
    for (int b = 0; b < kMaxB; ++b)
      if (b < nb)
#pragma unroll
        for (int u = 0; u < 2; ++u)
          gf[b][u] = *reinterpret_cast<const u32x4*>(grow + b * 64 + u * 32);
  }
  lds_barrier();

#pragma unroll
  for (int t = 0; t < kTok; ++t) {
    float tot = 0.f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) tot += red[t][w];
    const float inv = 1.0f / sqrtf(tot / static_cast<float>(a.H) + a.eps);
    const size_t row = static_cast<size_t>(t0 + t) * a.H;
#pragma unroll
    for (int c = 0; c < CPT; ++c) {
      const int ch = tid + c * kThreads;
      if (ch >= chunks) continue;
      u32x4* p = slot(t, ch);
      const u32x4 sum = *p;
      if (has_res && t < ntok)
        *reinterpret_cast<u32x4*>(static_cast<T*>(a.residual_out) + row +
                                  static_cast<size_t>(ch) * N) = sum;
      float v[N], wv[N], bv[N], o[N];
      Vec16<T>::unpack(sum, v);
      wc[c].unpack(wv);
      if (a.bias) bc[c].unpack(bv);
#pragma unroll
      for (int i = 0; i < N; ++i) {
        o[i] = v[i] * inv * wv[i];
        if (a.bias) o[i] += bv[i];
      }
      const u32x4 pk = pack16<T>(o);
      if (t < ntok)
        *reinterpret_cast<u32x4*>(static_cast<T*>(a.out) + row + static_cast<size_t>(ch) * N) = pk;
      *p = pk;
    }
  }
  lds_barrier();

  f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
  {
    const int cbase = wave * (a.H / 32);  // first chunk of the wave's quarter
#pragma unroll
    for (int b = 0; b < kMaxB; ++b)
      if (b < nb)
#pragma unroll
        for (int u = 0; u < 2; ++u)
          acc = pipe::Mfma16<T>::mma(*slot(r16 % kTok, cbase + 8 * b + 4 * u + kq), gf[b][u], acc);
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) part[wave][4 * kq + i][r16] = acc[i];
  lds_barrier();
  {
    const int t = tid / 16, e = tid % 16;
    if (t < kTok && t0 + t < a.T && e < ra.E) {
      float l = (part[0][t][e] + part[1][t][e]) + (part[2][t][e] + part[3][t][e]);
      if (ra.round_logits) l = to_f32(from_f32<T>(l));
      if (ra.bias) l += ra.bias[e];
      lg[t][e] = l;
      if (ra.logits_out) ra.logits_out[static_cast<size_t>(t0 + t) * ra.E + e] = l;
    }
  }
  lds_barrier();
  const int tt = tid / 16;
  if (tt < kTok && t0 + tt < a.T)
    group16_topk<1>(lg[tt], ra.E, ra.K, ra.renormalize, 0,
                    ra.topk_w + static_cast<size_t>(t0 + tt) * ra.out_ld,
                    ra.topk_ids + static_cast<size_t>(t0 + tt) * ra.out_ld, tid & 15);
}

template <typename T, typename W, int CPT>
hipError_t launch_norm_router_cpt(const NormArgs& a, const RouterArgs& ra, hipStream_t s) {
  const dim3 block(kThreads);
  // Two rows per workgroup from 512 rows on: the gate is then read from L2
  // once per two rows, and 256+ workgroups still fill the chip.
  if (a.T >= 512) {
    const dim3 grid((a.T + 1) / 2);
    if (ra.E <= 8)
      add_rmsnorm_router_kernel<T, W, CPT, 2, 8><<<grid, block, 0, s>>>(a, ra);
    else
      add_rmsnorm_router_kernel<T, W, CPT, 2, 16><<<grid, block, 0, s>>>(a, ra);
  } else {
    const dim3 grid(a.T);
    if (ra.E <= 8)
      add_rmsnorm_router_kernel<T, W, CPT, 1, 8><<<grid, block, 0, s>>>(a, ra);
    else
      add_rmsnorm_router_kernel<T, W, CPT, 1, 16><<<grid, block, 0, s>>>(a, ra);
  }
  return hipGetLastError();
}

template <typename T, typename W>
hipError_t launch_norm_router_mfma_tw(const NormArgs& a, const RouterArgs& ra, hipStream_t s) {
  const dim3 grid((a.T + kNormRouterRows - 1) / kNormRouterRows), block(kThreads);
  if (a.H <= 2048)
    add_rmsnorm_router_mfma_kernel<T, W, 1><<<grid, block, 0, s>>>(a, ra);
  else
    add_rmsnorm_router_mfma_kernel<T, W, 2><<<grid, block, 0, s>>>(a, ra);
  return hipGetLastError();
}

template <typename T>
hipError_t launch_norm_router_mfma_t(const NormArgs& a, const RouterArgs& ra, hipStream_t s) {
  if (a.weight_dtype == MOE355_BF16) return launch_norm_router_mfma_tw<T, bf16>(a, ra, s);
  if (a.weight_dtype == MOE355_F16) return launch_norm_router_mfma_tw<T, f16>(a, ra, s);
  return launch_norm_router_mfma_tw<T, float>(a, ra, s);
}

template <typename T, typename W>
hipError_t launch_norm_router_tw(const NormArgs& a, const RouterArgs& ra, hipStream_t s) {
  const int per_thread = (a.H / Vec16<T>::N + kThreads - 1) / kThreads;
  if (per_thread <= 1) return launch_norm_router_cpt<T, W, 1>(a, ra, s);
  if (per_thread <= 2) return launch_norm_router_cpt<T, W, 2>(a, ra, s);
  return launch_norm_router_cpt<T, W, 4>(a, ra, s);
}

template <typename T>
hipError_t launch_norm_router_t(const NormArgs& a, const RouterArgs& ra, hipStream_t s) {
  if (a.weight_dtype == MOE355_BF16) return launch_norm_router_tw<T, bf16>(a, ra, s);
  if (a.weight_dtype == MOE355_F16) return launch_norm_router_tw<T, f16>(a, ra, s);
  return launch_norm_router_tw<T, float>(a, ra, s);
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

// The fused kernel reads the gate from L2 once per one or two rows, the
// separate MFMA router once per 16 rows: fused wins while T * E stays small
// (Mixtral H=4096 E=8: 12.7 against 16.4 us at T=1024, even at T=2048 and
// 4096; 64 experts H=2048: 58 against 26 us at T=4096), and at decode sizes
// it saves a launch (8 against 14 us per call at T=1..256). Over more than 16
// experts one workgroup per token pulls the whole gate through one CU (256 KB
// at 64 experts, H=2048: 13.6 us at T=1), so given a logits buffer the split
// router, which spreads a token's experts over workgroups, runs instead.
bool norm_router_fusable(int T, int H, int E, int dtype, bool has_logits) {
  return (dtype == MOE355_BF16 || dtype == MOE355_F16) && E >= 1 && E <= kMaxRouterExperts &&
         H % 8 == 0 && H <= 4 * kThreads * 8 && T >= 1 &&
         static_cast<long long>(T) * E <= 8192 && (E <= 16 || !has_logits);
}

hipError_t launch_add_rmsnorm_router(const NormArgs& a, const RouterArgs& ra, int dtype,
                                     hipStream_t s) {
  if (a.T == 0) return hipSuccess;
  if (dtype == MOE355_BF16) return launch_norm_router_t<bf16>(a, ra, s);
  return launch_norm_router_t<f16>(a, ra, s);
}

bool norm_router_mfma_fusable(int T, int H, int E, int K, int dtype) {
  return (dtype == MOE355_BF16 || dtype == MOE355_F16) && E >= 1 && E <= 16 && K >= 1 &&
         K <= 8 && H >= 256 && H % 256 == 0 && H <= 4096 && T >= kNormRouterMfmaMinRows;
}

hipError_t launch_add_rmsnorm_router_mfma(const NormArgs& a, const RouterArgs& ra, int dtype,
                                          hipStream_t s) {
  if (a.T == 0) return hipSuccess;
  if (dtype == MOE355_BF16) return launch_norm_router_mfma_t<bf16>(a, ra, s);
  return launch_norm_router_mfma_t<f16>(a, ra, s);
}

hipError_t launch_add_rmsnorm(const NormArgs& a, int dtype, hipStream_t s) {
  if (a.T == 0) return hipSuccess;
  if (dtype == MOE355_BF16) return launch_norm_t<bf16>(a, s);
  if (dtype == MOE355_F16) return launch_norm_t<f16>(a, s);
  return launch_norm_t<float>(a, s);
}

}  // namespace moe355
