// Helpers of the LDS-pipelined MFMA grouped GEMM (ffn_tiled.hip): direct-to-LDS
// buffer loads, vmcnt-bounded workgroup barriers, the 32x32x16 MFMA, the work
// item decode and the tail split.
#pragma once

#include "common.h"

namespace moe355 {
namespace pipe {

typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(4))) int32_t const_i32;

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

// v unchanged, but opaque to the optimiser: per-lane indices derived from it
// are recomputed where they are used instead of being hoisted out of the
// persistent loop and kept live (or spilled to scratch, whose reloads wait on
// vmcnt and so drain the load pipeline) across the MFMA stream.
__device__ __forceinline__ int opaque(int v) {
  asm volatile("" : "+v"(v));
  return v;
}

// Direct-to-LDS loads through a buffer resource over [base, base + 2 GB - 1):
// an offset at or past kPadOffset is out of range, and the hardware's range
// check makes such a load write zeros to LDS without touching memory. Token
// rows past the end of a group (tile padding) load that way, so the MFMAs
// on padding multiply zeros: the results are discarded either way, but zero
// operands draw far less power, and the tiled kernels run at a power-limited
// clock (Mixtral-shape gate_up: 1.73 ms with random tokens, 1.24 ms with all
// tokens zero).
constexpr uint32_t kPadOffset = 0x80000000u;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t lds_rsrc(const void* base,
                                                         int num_records = 0x7fffffff) {
  // Raw buffer (stride 0); dword 3 sets a 32-bit data format, without which
  // gfx9 treats every untyped buffer access as out of range. num_records -1
  // (4 GB - 1) serves sources addressed by full 32-bit offsets (weights).
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, num_records, 0x00020000);
}

// One 1 KB direct-to-LDS load per wave from a buffer resource: lane i's 16
// bytes at byte offset off + soff of the resource land at dst + 16 i (zeros
// when off is out of range). soff is wave-uniform (an SGPR operand), so a
// load whose per-lane offset stays fixed over a K walk needs no address
// arithmetic: in a probe of 16 MFMAs plus 2-8 such loads per wave the loads
// cost ~24 cycles per 16 MFMAs in all, against ~17 cycles each for
// global_load_lds with its 64-bit per-lane address.
__device__ __forceinline__ void dma16_rsrc(__amdgpu_buffer_rsrc_t r, uint32_t off, uint32_t soff,
                                           uint8_t* dst) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void*)(dst), 16, off, soff, 0, 0);
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

template <typename T>
struct Mfma16;

template <>
struct Mfma16<bf16> {
  __device__ __forceinline__ static f32x4 mma(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
};

template <>
struct Mfma16<f16> {
  __device__ __forceinline__ static f32x4 mma(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
};

// One work item of the persistent grouped-GEMM kernels.
struct Tile {
  int split, wtile, e, row0, row_end;
  int height;  // rows per token tile of this expert (row_end - row0 <= height)
};

// Work item L of (split, weight tile, token tile), token tiles of tile_rows
// rows from the permute's tile map.
__device__ __forceinline__ Tile decode_tile(const FfnArgs& a, int L, int per_split, int n_t,
                                            int tile_rows) {
  // L is wave-uniform; saying so keeps the tile-map reads on the scalar unit
  // (vector loads here would be waited for with vmcnt and drain the
  // direct-to-LDS pipeline at every item boundary).
  // The tables are read through the constant address space (they do not
  // change during the kernel), so the compiler may use scalar loads although
  // the kernel stores to memory it cannot tell apart from them.
  L = __builtin_amdgcn_readfirstlane(L);
  const const_i32* tile_map = (const const_i32*)(a.tile_map);
  const const_i32* offsets = (const const_i32*)(a.offsets);
  Tile t;
  t.split = L / per_split;
  const int rem = L - t.split * per_split;
  if (a.group_t < 0) {
    // One group per expert: its token tiles x all weight tiles, the token tile
    // varying fastest. The group of item rem starts at the first tile b of the
    // expert owning tile rem / n_wtiles (tiles of an expert are consecutive
    // and its tile height apart, so b follows from that tile's first row).
    const int t0 = rem / a.n_wtiles;
    const int e = tile_map[2 + 2 * t0];
    const int eb = offsets[e], ee = offsets[e + 1];
    const int h = tile_height(ee - eb, tile_rows);
    const int b = t0 - (tile_map[3 + 2 * t0] - eb) / h;
    const int ne = (ee - eb + tile_rows - 1) / tile_rows;
    const int r2 = rem - b * a.n_wtiles;
    t.wtile = r2 / ne;
    const int tt = b + (r2 - t.wtile * ne);
    t.e = e;
    t.height = h;
    t.row0 = tile_map[3 + 2 * tt];
    t.row_end = min(t.row0 + h, ee);
    return t;
  }
  // Items come in groups of gt token tiles x all weight tiles, the token tile
  // varying fastest inside a group; the last group may hold fewer token tiles.
  const int gfull = a.group_t > 0 ? a.group_t : n_t;
  const int g = rem / (gfull * a.n_wtiles);
  const int r2 = rem - g * gfull * a.n_wtiles;
  const int gt = min(gfull, n_t - g * gfull);
  t.wtile = r2 / gt;
  const int tt = g * gfull + (r2 - t.wtile * gt);
  t.e = tile_map[2 + 2 * tt];
  t.row0 = tile_map[3 + 2 * tt];
  t.height = tile_height(offsets[t.e + 1] - offsets[t.e], tile_rows);
  t.row_end = min(t.row0 + t.height, offsets[t.e + 1]);
  return t;
}

// Tail split of a persistent grouped GEMM. With n_work items on G workgroups
// the last n_work % G items (the tail) would run alone while the other CUs
// idle for a whole item. Instead each tail item is cut along K into S parts
// (S a power of two, S | nk, S * tail <= cap), one unit per idle workgroup,
// whose fp32 partial tiles a fix-up pass sums. Items [0, n_full) run whole;
// unit u < n_units is k-part u % S of item n_full + u / S. S minimises
// 14 * nk / S + S * tail: a 64-k step of a 256x256 tile costs about fourteen
// times what one unit's partial tile costs to write and read back through HBM
// (so a short K or a wide tail keeps the item whole). cap = 0 disables the
// split.
struct WorkSplit {
  int n_full, n_units, S;
};

__device__ __forceinline__ WorkSplit work_split(int n_work, int G, int nk, int cap) {
  WorkSplit w{n_work, 0, 1};
  const int R = G > 0 ? n_work / G : 0, tail = n_work - R * G;
  if (cap <= 0 || tail == 0) return w;
  cap = min(cap, G);
  int best = 14 * nk;
  for (int s = 2; s <= 16 && s * tail <= cap && nk % s == 0; s *= 2) {
    const int c = 14 * nk / s + s * tail;
    if (c < best) {
      best = c;
      w.S = s;
    }
  }
  if (w.S > 1) {
    w.n_full = R * G;
    w.n_units = tail * w.S;
  }
  return w;
}

}  // namespace pipe
}  // namespace moe355
