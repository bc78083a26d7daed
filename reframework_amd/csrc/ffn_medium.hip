// Grouped expert FFN on bf16/f16 MFMA for medium groups (tens to a few hundred
// rows per expert).
//
// Replaces the same per-expert GEMMs as ffn_tiled.hip (reframework/moe/
// fused.py:76-83) when groups are too large for the skinny kernel but would
// leave most of a 256-token tile empty: Mixtral at 256 tokens (64 rows per
// expert), skewed routing, fine-grained experts. A work item is 256 weight
// rows x 64 token rows, so padding costs at most 63 rows per expert; the layer
// is then bound by streaming each routed expert's weights from HBM.
//
// Four waves side by side along the weight rows, each owning 2x2 blocks of
// v_mfma_f32_32x32x16 (64 weight rows x 64 tokens, 64 fp32 accumulators).
//   gate_up: wave w's two weight blocks are gate rows 32w..32w+31 of the tile
//            and the matching up rows, so silu(g)*u is applied in registers.
//   down:    wave w owns w2 rows 64w..64w+63 of the tile; fp32 partials per
//            K-split into y.
// Pipeline as in the 256-row kernel: 32 k per step, direct-to-LDS loads (20 x
// 1 KB per step, 5 per wave), eight 20 KB LDS buffers, loads issued seven steps
// ahead, a mid-step barrier that waits only for the next step, and persistent
// workgroups (one per CU) whose K-steps stream across work items.
#include "dma_pipe.h"

namespace moe355 {
namespace {

using namespace pipe;

constexpr int kThreads = 256;
constexpr int kTileW = 256;
constexpr int kTileT = 64;
constexpr int kWRegion = kTileW * kRowBytes;       // 16 KB
constexpr int kStageBytes = kWRegion + kTileT * kRowBytes;  // 20 KB
constexpr int kStages = 8;
constexpr int kLdsBytes = kStages * kStageBytes;   // 160 KB
constexpr int kLPW = kStageBytes / 1024 / 4;       // 5 loads of 1 KB per wave per step
constexpr int kHalf0 = 3;                          // of them issued in the first half-step
constexpr int kWLoads = kWRegion / 1024;           // loads 0..15 fill the weight region

template <typename T, bool kGateUp>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(1, 1)))
void ffn_medium_kernel(const FfnArgs a) {
  __shared__ __attribute__((aligned(1024))) uint8_t lds[kLdsBytes];

  const int tid = threadIdx.x, lane = tid & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);

  const int n_t = a.tile_map[0];
  const int per_split = a.n_wtiles * n_t;
  const int n_work = a.splits * per_split;
  const int G = gridDim.x;
  int Lc = xcd_remap(blockIdx.x, G);  // work item being multiplied
  if (Lc >= n_work) return;

  const int ld = kGateUp ? a.H : a.I;  // elements per weight row and per token row
  const uint32_t pitch = static_cast<uint32_t>(ld * 2);
  const int nk = a.k_per_split / kBK;
  auto decode = [&](int L) { return decode_tile(a, L, per_split, n_t, kTileT); };

  // Load q of this wave is stage load li = 5 * wave + q; it fills 16 rows of
  // 64 B at LDS offset li * 1 KB: weight rows 16 li.. for li < 16, token rows
  // 16 (li - 16).. after. Lane i covers row 16 * blk + i / 4, physical chunk
  // i % 4, i.e. that row's logical chunk swz(i % 4, row).
  auto load_row = [&](int q) { return ((kLPW * wave + q) & 15) * 16 + (lane >> 2); };
  auto is_tok = [&](int q) { return kLPW * wave + q >= kWLoads; };

  int grow[kLPW];  // gate_up token loads: x rows of the next work item (row_src)
  auto fetch_rows = [&](const Tile& t) {
#pragma unroll
    for (int q = 0; q < kLPW; ++q)
      if (kGateUp && is_tok(q)) grow[q] = a.row_src[min(t.row0 + load_row(q), t.row_end - 1)];
  };

  int Ll = Lc, lkt = 0;         // load cursor
  __amdgpu_buffer_rsrc_t lw;    // weight source of the load cursor's item
  __amdgpu_buffer_rsrc_t lx;    // token source
  uint32_t lgoff[kLPW];
  auto setup_load = [&](const Tile& t) {
    const size_t kbeg = static_cast<size_t>(t.split) * a.k_per_split;
    lw = lds_rsrc(static_cast<const char*>(a.w[t.e]) + kbeg * 2, -1);
    lx = lds_rsrc(kGateUp ? static_cast<const char*>(a.x) + kbeg * 2
                          : static_cast<const char*>(a.x) +
                                (static_cast<size_t>(t.row0) * ld + kbeg) * 2);
#pragma unroll
    for (int q = 0; q < kLPW; ++q) {
      const int r = load_row(q);
      int src_row;
      uint32_t pad = 0;
      if (!is_tok(q)) {
        src_row = kGateUp ? (r < kTileW / 2 ? t.wtile * (kTileW / 2) + r
                                            : a.I + t.wtile * (kTileW / 2) + (r - kTileW / 2))
                          : t.wtile * kTileW + r;
      } else {
        src_row = kGateUp ? grow[q] : min(t.row0 + r, t.row_end - 1) - t.row0;
        // Token rows past the group's end load zeros (out of the resource's
        // range), OR-ed in rather than selected (see the tiled kernel).
        pad = t.row0 + r < t.row_end ? 0u : kPadOffset;
      }
      lgoff[q] = (static_cast<uint32_t>(src_row) * pitch + swz(lane & 3, r) * 16) | pad;
    }
  };
  auto prefetch_next_rows = [&]() {
    if (kGateUp && Ll + G < n_work) fetch_rows(decode(Ll + G));
  };
  // Past the last work item the cursor stays on its final step: the tail
  // keeps issuing in-bounds loads into buffers nobody reads, so the vmcnt
  // accounting of the pipeline stays fixed.
  auto advance_load = [&]() {
    if (++lkt < nk) return;
    if (Ll + G < n_work) {
      Ll += G;
      lkt = 0;
      setup_load(decode(Ll));
      prefetch_next_rows();
    } else {
      lkt = nk - 1;
    }
  };
  auto issue = [&](uint8_t* lb, int q) {
    dma16_rsrc(is_tok(q) ? lx : lw, lgoff[q], lkt * kRowBytes, lb + (kLPW * wave + q) * 1024);
  };

  // MFMA operand rows of this wave inside a stage.
  const int lr = lane & 31, kh = lane >> 5;
  uint32_t arow[2], brow[2];
#pragma unroll
  for (int b = 0; b < 2; ++b) {
    const int rw = kGateUp ? b * (kTileW / 2) + 32 * wave : 64 * wave + 32 * b;
    arow[b] = (rw + lr) * kRowBytes;
    brow[b] = kWRegion + (32 * b + lr) * kRowBytes;
  }
  uint32_t coff[kBK / 16];
#pragma unroll
  for (int ks = 0; ks < kBK / 16; ++ks) coff[ks] = swz(ks * 2 + kh, lr) << 4;

  f32x16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = f32x16{};

  // Invariant at the top of step g: step g is in LDS and visible to every
  // wave, its sub-step 0 operands are in registers, and the loads of steps
  // g+1 .. g+kStages-2 are in flight. Step g issues step g+kStages-1 into the
  // buffer of step g-1 (whose last reads finished before step g-1's mid-step
  // barrier); the mid-step barrier waits for step g+1 only. Other vector-
  // memory operations (row_src prefetch, epilogue stores) only make the waits
  // stricter.
  {
    const Tile t0 = decode(Ll);
    if (kGateUp) fetch_rows(t0);
    setup_load(t0);
    prefetch_next_rows();
  }
#pragma unroll
  for (int s = 0; s < kStages - 1; ++s) {
#pragma unroll
    for (int q = 0; q < kLPW; ++q) issue(lds + s * kStageBytes, q);
    advance_load();
  }
  dma_barrier<(kStages - 2) * kLPW>();  // step 0 landed

  u32x4 fa[2][2], fb[2][2];
#pragma unroll
  for (int b = 0; b < 2; ++b) {
    fa[0][b] = *reinterpret_cast<const u32x4*>(lds + arow[b] + coff[0]);
    fb[0][b] = *reinterpret_cast<const u32x4*>(lds + brow[b] + coff[0]);
  }
  wait_lgkm0();

  // Half-step: wait for its operands, 4 MFMAs, and the other half's 4 operand
  // reads plus this half's loads interleaved with them.
  auto half = [&](const u32x4* af, const u32x4* bf, const uint8_t* src, int ks, u32x4* na,
                  u32x4* nb, uint8_t* lb, int q0, int nq) {
    wait_lgkm0();
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) acc[i][j] = Mfma32<T>::mma(af[i], bf[j], acc[i][j]);
    // Memory operations in schedule order (the compiler keeps LDS reads and
    // direct-to-LDS loads in program order).
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      na[i] = *reinterpret_cast<const u32x4*>(src + arow[i] + coff[ks]);
      if (i < nq) issue(lb, q0 + i);
      nb[i] = *reinterpret_cast<const u32x4*>(src + brow[i] + coff[ks]);
    }
    if (nq > 2) issue(lb, q0 + 2);
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // LDS read
      __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // global -> LDS load
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
    __builtin_amdgcn_sched_barrier(0);
  };

  int cb = 0;  // LDS buffer of the step being multiplied
  Tile ct = decode(Lc);
  while (true) {
    for (int kt = 0; kt < nk; ++kt) {
      const int nb_ = cb == kStages - 1 ? 0 : cb + 1;
      const int lb_ = cb == 0 ? kStages - 1 : cb - 1;  // (cb + kStages - 1) % kStages
      uint8_t* st = lds + cb * kStageBytes;
      uint8_t* nx = lds + nb_ * kStageBytes;
      uint8_t* lb = lds + lb_ * kStageBytes;
      half(fa[0], fb[0], st, 1, fa[1], fb[1], lb, 0, kHalf0);
      wait_lgkm0();
      dma_barrier<(kStages - 3) * kLPW + kHalf0>();  // step g+1 landed
      half(fa[1], fb[1], nx, 0, fa[0], fb[0], lb, kHalf0, kLPW - kHalf0);
      advance_load();
      cb = nb_;
    }

    // Epilogue. Lane (lr, kh) of block (i, j) holds, for q = 0..3, features
    // 8q + 4kh + 0..3 of weight block i and token 32j + lr of the tile.
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int prow = ct.row0 + 32 * j + lr;
      if (prow >= ct.row_end) continue;
      if (kGateUp) {
        T* inter = static_cast<T*>(a.out) + static_cast<size_t>(prow) * a.I;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int col = ct.wtile * (kTileW / 2) + 32 * wave + 8 * q + 4 * kh;
          float v[4];
#pragma unroll
          for (int r = 0; r < 4; ++r)
            v[r] = gate_act_fast(a.act, acc[0][j][4 * q + r]) * acc[1][j][4 * q + r];
          store4<T>(inter + col, v[0], v[1], v[2], v[3]);
        }
      } else {
        float* y = static_cast<float*>(a.out) + static_cast<size_t>(ct.split) * a.R * a.H +
                   static_cast<size_t>(prow) * a.H;
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const int h = ct.wtile * kTileW + 64 * wave + 32 * i + 8 * q + 4 * kh;
            store4<float>(y + h, acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2],
                          acc[i][j][4 * q + 3]);
          }
      }
    }

#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) acc[i][j] = f32x16{};
    Lc += G;
    if (Lc >= n_work) break;
    ct = decode(Lc);
  }
  // No direct-to-LDS write may still be in flight when the workgroup's LDS is
  // released.
  wait_vmcnt<0>();
}

template <bool kGateUp>
hipError_t launch_medium(const FfnArgs& a, int dtype, hipStream_t s) {
  const long work = static_cast<long>(a.n_wtiles) * a.max_tiles * a.splits;
  if (work == 0) return hipSuccess;
  const int cus = device_cu_count();
  const int nwg = static_cast<int>(work < cus ? work : cus);
  if (dtype == MOE355_BF16)
    ffn_medium_kernel<bf16, kGateUp><<<dim3(nwg), dim3(kThreads), 0, s>>>(a);
  else
    ffn_medium_kernel<f16, kGateUp><<<dim3(nwg), dim3(kThreads), 0, s>>>(a);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_gate_up_medium(const FfnArgs& a, int dtype, hipStream_t s) {
  return launch_medium<true>(a, dtype, s);
}

hipError_t launch_down_medium(const FfnArgs& a, int dtype, hipStream_t s) {
  return launch_medium<false>(a, dtype, s);
}

}  // namespace moe355
