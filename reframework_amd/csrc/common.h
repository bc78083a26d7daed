// Shared device types, conversions and launcher declarations of libmoe355.
//
// Everything here is gfx950 (CDNA4) code: 64-lane wavefronts, bf16/f16 MFMA,
// 160 KB of LDS per CU. Storage types are the raw 16-bit formats; all
// arithmetic accumulates in fp32.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include <type_traits>

#include "../../include/moe355.h"

namespace moe355 {

typedef __bf16 bf16;
typedef _Float16 f16;

typedef bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef f16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kWave = 64;
constexpr int kMaxExperts = MOE355_MAX_EXPERTS;
constexpr int kPermuteChunk = 256;       // routed slots per block of the count + scatter launches
constexpr int kPermuteSingleMax = 1024;  // up to this many slots one block does the whole permute

// ---------------------------------------------------------------- conversions
template <typename T>
__device__ __forceinline__ float to_f32(T v) {
  return static_cast<float>(v);
}

template <typename T>
__device__ __forceinline__ T from_f32(float v) {
  return static_cast<T>(v);  // round-to-nearest-even for bf16 and f16
}

// Unpack a 16-byte vector of storage elements to fp32.
template <typename T>
struct Vec16;

template <>
struct Vec16<float> {
  static constexpr int N = 4;
  __device__ __forceinline__ static void unpack(u32x4 v, float* o) {
    o[0] = __uint_as_float(v.x);
    o[1] = __uint_as_float(v.y);
    o[2] = __uint_as_float(v.z);
    o[3] = __uint_as_float(v.w);
  }
};

template <>
struct Vec16<bf16> {
  static constexpr int N = 8;
  __device__ __forceinline__ static void unpack(u32x4 v, float* o) {
    uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      o[2 * i] = __uint_as_float(w[i] << 16);
      o[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
    }
  }
};

template <>
struct Vec16<f16> {
  static constexpr int N = 8;
  __device__ __forceinline__ static void unpack(u32x4 v, float* o) {
    f16x8 h = __builtin_bit_cast(f16x8, v);
#pragma unroll
    for (int i = 0; i < 8; ++i) o[i] = static_cast<float>(h[i]);
  }
};

// Pack four fp32 values into four storage elements (8 bytes for 16-bit types).
template <typename T>
__device__ __forceinline__ void store4(T* dst, float a, float b, float c, float d) {
  dst[0] = from_f32<T>(a);
  dst[1] = from_f32<T>(b);
  dst[2] = from_f32<T>(c);
  dst[3] = from_f32<T>(d);
}

template <>
__device__ __forceinline__ void store4<bf16>(bf16* dst, float a, float b, float c, float d) {
  typedef bf16 bf16x4 __attribute__((ext_vector_type(4)));
  bf16x4 v = {from_f32<bf16>(a), from_f32<bf16>(b), from_f32<bf16>(c), from_f32<bf16>(d)};
  *reinterpret_cast<bf16x4*>(dst) = v;
}

template <>
__device__ __forceinline__ void store4<f16>(f16* dst, float a, float b, float c, float d) {
  typedef f16 f16x4 __attribute__((ext_vector_type(4)));
  f16x4 v = {from_f32<f16>(a), from_f32<f16>(b), from_f32<f16>(c), from_f32<f16>(d)};
  *reinterpret_cast<f16x4*>(dst) = v;
}

template <>
__device__ __forceinline__ void store4<float>(float* dst, float a, float b, float c, float d) {
  *reinterpret_cast<f32x4*>(dst) = f32x4{a, b, c, d};
}

// ---------------------------------------------------------------- activations
// Gated activations of reframework/layers/activation.py:15-59 applied to the
// gate half: silu(g) = g * sigmoid(g); gelu(g) = g/2 * (1 + erf(g/sqrt2));
// gelu_tanh(g) = g/2 * (1 + tanh(sqrt(2/pi) * (g + 0.044715 g^3))).
__device__ __forceinline__ float gate_act(int act, float g) {
  if (act == MOE355_ACT_SILU) return g / (1.0f + expf(-g));
  if (act == MOE355_ACT_GELU) return 0.5f * g * (1.0f + erff(g * 0.70710678118654752f));
  const float c = 0.79788456080286536f;  // sqrt(2/pi)
  return 0.5f * g * (1.0f + tanhf(c * (g + 0.044715f * g * g * g)));
}

// sigmoid(z) = 1 / (1 + e^-z) as 1 / (1 + 2^(-z log2 e)) on the hardware
// transcendental unit (v_exp_f32, v_rcp_f32; ~1 ulp each). Limits: z -> -inf
// gives 2^+inf = inf and rcp(inf) = 0; z -> +inf gives 2^-inf = 0 and 1.
__device__ __forceinline__ float sigmoid_hw(float z) {
  return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(z * -1.4426950408889634f));
}

// gate_act for the 16-bit (bf16/f16) kernels, whose outputs are rounded to 8
// or 11 significant bits: the relative error of sigmoid_hw (~3e-7) is far below
// that rounding, and the precise expf and IEEE division of gate_act cost about
// 30 VALU instructions per element in an epilogue that keeps the MFMA pipe
// idle. silu(g) = g * sigmoid(g); gelu_tanh(g) = g/2 * (1 + tanh(u)) =
// g * sigmoid(2u) with u = sqrt(2/pi) * (g + 0.044715 g^3); erf-gelu keeps erff.
__device__ __forceinline__ float gate_act_fast(int act, float g) {
  if (act == MOE355_ACT_SILU) return g * sigmoid_hw(g);
  if (act == MOE355_ACT_GELU) return 0.5f * g * (1.0f + erff(g * 0.70710678118654752f));
  const float c2 = 1.5957691216057308f;  // 2 sqrt(2/pi)
  return g * sigmoid_hw(c2 * (g + 0.044715f * g * g * g));
}

// gate_act_fast with SiLU resolved at compile time (kSilu) for epilogues that
// pick the activation once per tile.
template <bool kSilu>
__device__ __forceinline__ float gate_act_16(int act, float g) {
  return kSilu ? g * sigmoid_hw(g) : gate_act_fast(act, g);
}

// ---------------------------------------------------------------- wave helpers
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
  return v;
}

// Rows per token tile of an expert of n rows in a tile map of tile_rows-row
// tiles. 256-row tiles share the expert's rows evenly over its ceil(n / 256)
// tiles, the height rounded up to the 32-row token-block pair the 256-row
// GEMM multiplies (1085 rows: 5 tiles of 224 rows, the last 189); the other
// tile maps are tile_rows apart. The tile count is ceil(n / tile_rows) either
// way.
__host__ __device__ __forceinline__ int tile_height(int n, int tile_rows) {
  if (tile_rows != 256 || n <= 0) return tile_rows;
  const int nt = (n + 255) / 256;
  return (((n + nt - 1) / nt) + 31) & ~31;
}

// Map a flat workgroup id so that ids dispatched to the same XCD (the hardware
// deals workgroups round-robin over the 8 XCDs) get consecutive logical ids.
// Tiles that share a weight slab then run on one XCD and share its L2.
__device__ __forceinline__ int xcd_remap(int pid, int nwg) {
  const int xcd = pid & 7, slot = pid >> 3;
  const int q = nwg >> 3, rem = nwg & 7;
  const int base = xcd < rem ? xcd * (q + 1) : rem * (q + 1) + (xcd - rem) * q;
  return base + slot;
}

// ---------------------------------------------------------------- kernel args
struct RouterArgs {
  const void* x;        // [T,H] or nullptr when logits_in is given
  const void* gate;     // [E,H]
  const float* bias;    // [E] or nullptr
  const float* logits_in;  // [T,E] fp32 (topk_from_logits mode)
  float* logits_out;    // [T,E] or nullptr
  float* topk_w;        // [T,K]
  int32_t* topk_ids;    // [T,K]
  int T, H, E, K;
  int renormalize, round_logits, entropy_k_min;
  int out_ld;           // row stride of topk_w / topk_ids (>= K)
};

struct PermuteArgs {
  const void* ids;       // [R] int32 or int64
  int32_t* block_counts; // [n_blocks, E]
  int32_t* offsets;      // [E+1]
  int32_t* slot_to_row;  // [R]
  int32_t* row_src;      // [R]
  int32_t* tile_map;     // [2 + 2*max_tiles]
  int R, K, E, n_blocks, tile_rows, max_tiles;
  int ids_int64, map_len;  // map_len 0: no map
  int32_t map[kMaxExperts];
  const float* weights;    // [R] routing weights, or nullptr: a slot of weight 0 is dropped
};

// Local expert of routed slot `slot`, or -1 when the slot is dropped (an id
// the optional map sends negative or outside [0, E), or that lies outside the
// map; with weights, a slot of weight exactly 0, which would add 0 * y).
__device__ __forceinline__ int routed_expert(const PermuteArgs& a, int slot) {
  if (a.weights && a.weights[slot] == 0.0f) return -1;
  long long id = a.ids_int64 ? static_cast<const int64_t*>(a.ids)[slot]
                             : static_cast<long long>(static_cast<const int32_t*>(a.ids)[slot]);
  if (a.map_len > 0) {
    if (id < 0 || id >= a.map_len) return -1;
    id = a.map[id];
  }
  return (id >= 0 && id < a.E) ? static_cast<int>(id) : -1;
}

struct FfnArgs {
  const void* x;           // gate_up: tokens [T,H]; down: inter [R,I]
  const int32_t* row_src;  // [R]
  const int32_t* tile_map; // [2 + 2*max_tiles]
  const int32_t* offsets;  // [E+1]
  void* out;               // gate_up: inter [R,I]; down: y [S,R,H] fp32, or [R,H] in the layer dtype (y16)
  int H, I, R;
  int max_tiles, n_wtiles, splits, k_per_split;
  int act;
  float* part;             // tiled gate_up: tail-split partial tiles, part_units x 256 KB
  int part_units;          // capacity of part in 256x256 fp32 tiles (0: no tail split)
  int grid;                // workgroups of the tiled launch (the fix-up recomputes its split)
  int group_t;             // token tiles per item group (0: all; -1: one group per expert; see decode_tile)
  int tile_rows;           // token rows per tile of the tile map (tiled kernels: 256, or 128 for half tiles)
  int y16;                 // tiled down with one K-split: y rounded to the layer dtype
  int ragged;              // full-tile kernel: per-item token-block count and rotated XCD slots
  const void* w[kMaxExperts];  // w1[e] ([2I,H]) or w2[e] ([H,I])
  // Skinny gate_up only, when self_permute: every workgroup groups the <= 64
  // routed slots of perm itself (no permute launch), and workgroup 0 writes
  // perm's offsets, slot_to_row, row_src and tile_map for the later stages.
  int self_permute;
  PermuteArgs perm;
};

struct NormArgs {
  const void* x;        // [T,H]
  const void* residual; // [T,H] added to x, or nullptr for a plain norm of x
  void* residual_out;   // [T,H] x + residual (may alias residual or x)
  const void* weight;   // [H] (weight_dtype)
  const void* bias;     // [H] (weight_dtype) or nullptr
  void* out;            // [T,H] normed
  int T, H, weight_dtype;
  float eps;
};

struct CombineArgs {
  const void* y;             // [S,R,H] fp32, or [R,H] in the layer dtype (y16)
  const float* topk_w;       // [T,K]
  const int32_t* slot_to_row;  // [T*K]
  void* out;                 // [T,H]
  int T, K, H, R, splits;
  int accumulate;
  int y16;
};

// Compute units of the current device (256 when it cannot be queried, e.g. on a
// host without a GPU); cached per device.
int device_cu_count();

// ---------------------------------------------------------------- launchers
// Each returns the hipError_t of the launch (hipSuccess when nothing to do).
hipError_t launch_router(const RouterArgs& a, int dtype, hipStream_t s);
hipError_t launch_add_rmsnorm(const NormArgs& a, int dtype, hipStream_t s);
int norm_max_hidden(int dtype);
hipError_t launch_topk_from_logits(const RouterArgs& a, hipStream_t s);
hipError_t launch_permute(const PermuteArgs& a, hipStream_t s);
hipError_t launch_gate_up_tiled(const FfnArgs& a, int dtype, hipStream_t s);
hipError_t launch_down_tiled(const FfnArgs& a, int dtype, hipStream_t s);
hipError_t launch_gate_up_skinny(const FfnArgs& a, int dtype, hipStream_t s);
hipError_t launch_down_skinny(const FfnArgs& a, int dtype, hipStream_t s);
hipError_t launch_gate_up_simt(const FfnArgs& a, int dtype, hipStream_t s);
hipError_t launch_down_simt(const FfnArgs& a, int dtype, hipStream_t s);
hipError_t launch_combine(const CombineArgs& a, int out_dtype, hipStream_t s);
// Fused residual add + RMSNorm + router (norm.hip): 16-bit types, E <= 64,
// H a multiple of 8 up to 8192, T * E <= 8192, and E <= 16 where a logits
// buffer lets the split router run instead.
constexpr int kMaxRouterExperts = 64;
bool norm_router_fusable(int T, int H, int E, int dtype, bool has_logits);
// Prefill sizes (T >= kNormRouterMfmaMinRows, up to 16 experts): the one-launch
// norm + MFMA router, bit for bit the norm kernel followed by the MFMA router.
// It wins from ~2048 rows (H = 4096, 8 experts: 19.3 against 19.8 us at 2048,
// 28 against 31 us at 4096); below, the two launches of the split path are
// the faster.
constexpr int kNormRouterMfmaMinRows = 2048;
bool norm_router_mfma_fusable(int T, int H, int E, int K, int dtype);
hipError_t launch_add_rmsnorm_router_mfma(const NormArgs& a, const RouterArgs& ra, int dtype,
                                          hipStream_t s);
hipError_t launch_add_rmsnorm_router(const NormArgs& a, const RouterArgs& ra, int dtype,
                                     hipStream_t s);
hipError_t launch_cast_f32(const float* src, void* dst, size_t n, int dtype, hipStream_t s);
hipError_t launch_copy_bytes(const void* src, void* dst, size_t n, hipStream_t s);
// Up to four byte regions (16-byte aligned sources and destinations).
constexpr int kMaxCopyRegions = 4;
struct CopyRegions {
  const uint8_t* src[kMaxCopyRegions];
  uint8_t* dst[kMaxCopyRegions];
  size_t bytes[kMaxCopyRegions];
  int count;
};
hipError_t launch_copy_regions(const CopyRegions& r, hipStream_t s);
hipError_t launch_merge_host(const float* acc, const float* host, void* out, size_t n, int dtype,
                             hipStream_t s);

}  // namespace moe355
