// Helpers shared by the LDS-pipelined MFMA kernels (ffn_tiled.hip,
// ffn_medium.hip): 64-byte LDS rows swizzled in 16-byte chunks, direct-to-LDS
// global loads, vmcnt-bounded workgroup barriers and the 32x32x16 MFMA.
#pragma once

#include "common.h"

namespace moe355 {
namespace pipe {

constexpr int kBK = 32;             // k elements per pipeline step
constexpr int kRowBytes = kBK * 2;  // 64 B: 4 chunks of 16 B

// Physical 16-byte chunk of logical chunk c (0..3) in LDS row r (64 B). Four
// consecutive rows fill one 256-byte span of a 64-bank LDS; XOR with
// (r >> 2) & 3 gives the four such spans of any 16 consecutive rows different
// chunk columns, so 16 rows read at one logical chunk hit 16 distinct 16-byte
// bank groups. The map is an involution.
__device__ __forceinline__ uint32_t swz(int c, int r) {
  return static_cast<uint32_t>(c ^ ((r >> 2) & 3));
}

typedef __attribute__((address_space(3))) void lds_void;

// s_waitcnt that waits until at most n vector-memory operations are
// outstanding (gfx9 encoding: vmcnt in bits 3:0 and 15:14; expcnt and lgkmcnt
// left at their maxima, i.e. not waited on).
template <int n>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(n >= 0 && n < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8));
}

__device__ __forceinline__ void wait_lgkm0() { __builtin_amdgcn_s_waitcnt(0xc07f); }

// Workgroup barrier after which the direct-to-LDS loads older than the newest
// n of every wave are visible to all waves. __syncthreads() would wait for all
// vector-memory operations (vmcnt(0)), draining the load pipeline; the signal
// fences only stop the compiler from moving memory accesses across.
template <int n>
__device__ __forceinline__ void dma_barrier() {
  wait_vmcnt<n>();
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_barrier();
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// One 1 KB direct-to-LDS load per wave: lane i's 16 bytes land at dst + 16 i.
__device__ __forceinline__ void dma16(const void* src, uint8_t* dst) {
  __builtin_amdgcn_global_load_lds(src, (lds_void*)(dst), 16, 0, 0);
}

template <typename T>
struct Mfma32;

template <>
struct Mfma32<bf16> {
  __device__ __forceinline__ static f32x16 mma(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
};

template <>
struct Mfma32<f16> {
  __device__ __forceinline__ static f32x16 mma(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
};

// One work item of the persistent grouped-GEMM kernels.
struct Tile {
  int split, wtile, e, row0, row_end;
};

// Work item L of (split, weight tile, token tile), token tiles of tile_rows
// rows from the permute's tile map.
__device__ __forceinline__ Tile decode_tile(const FfnArgs& a, int L, int per_split, int n_t,
                                            int tile_rows) {
  Tile t;
  t.split = L / per_split;
  const int rem = L - t.split * per_split;
  t.wtile = rem / n_t;
  const int tt = rem - t.wtile * n_t;
  t.e = a.tile_map[2 + 2 * tt];
  t.row0 = a.tile_map[3 + 2 * tt];
  t.row_end = min(t.row0 + tile_rows, a.offsets[t.e + 1]);
  return t;
}

}  // namespace pipe
}  // namespace moe355
