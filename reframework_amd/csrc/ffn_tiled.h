// Grouped expert FFN on bf16/f16 MFMA, prefill-sized groups.
//
// Replaces the per-expert GEMMs of fused_experts (reframework/moe/fused.py:
// 76-83): `x @ w1[e].t()`, gated_act_and_mul, `inter @ w2[e].t()`. One launch
// covers every expert: work items are (K-split, weight tile, token tile) over
// the tile map written by the permute, so no host round trip decides group
// sizes.
//
// Tile: 256 weight rows x 256 token rows, 4 waves in a 2x2 arrangement, each
// wave owning 8x8 blocks of v_mfma_f32_16x16x32 (a 128x128 sub-tile, 256 fp32
// accumulators). An expert's token tiles share its rows evenly (tile_height),
// and the MFMAs multiply only the 32-row token-block pairs a tile needs. Weight rows are the MFMA M side and tokens the N side, so each
// lane ends up holding 4 consecutive output features of one token and stores
// them as one vector.
//   gate_up: the 256 weight rows are 128 gate rows and the 128 matching up
//            rows, so gate and up of the same (token, feature) land in the same
//            lane and silu(g)*u is applied in registers; token rows are
//            gathered straight from x through row_src (no permuted copy of x).
//   down:    256 rows of w2 against the permuted inter rows, fp32 partials
//            per K-split into y.
// Operands move global -> LDS with direct-to-LDS loads (no register staging)
// in steps of 64 k. One operand of one step is a 32 KB buffer of 256 rows of
// 128 B, so every load instruction fetches whole 128-byte lines (8 rows x
// 128 B): the L1 then tracks half as many outstanding requests per byte as with
// 64-byte rows, which is what bounds the load stream. Five such buffers (the
// whole 160 KB LDS) form a ring over the operand stream W0 X0 W1 X1 ...;
// weights are issued two steps ahead of their use, tokens (mostly L2 hits)
// one step ahead. Rows are XOR-swizzled in 16-byte chunks (swz8) so the MFMA
// operand reads are bank-conflict free. The kernel is persistent (one
// workgroup per CU) and streams its steps across tile boundaries, so each
// tile's pipeline fill overlaps the previous tile's epilogue. The items left
// for a last, mostly idle round are split along K over the idle CUs
// (work_split); their fp32 partial tiles are summed (and, for gate_up,
// activated) by the fix-up kernels. 128-row token tiles run
// ffn_tiled_half_kernel, the same scheme on v_mfma_f32_32x32x16 with its loads
// split between waves (described there).
#pragma once
#include "acc_regs.h"
#include "dma_pipe.h"

namespace moe355 {
namespace {

using namespace pipe;

constexpr int kThreads = 256;
constexpr int kTileW = 256;
constexpr int kTileT = 256;
constexpr int kSK = 64;                         // k per pipeline step
constexpr int kSRowBytes = kSK * 2;             // 128 B: 8 chunks of 16 B
constexpr int kBufBytes = kTileW * kSRowBytes;  // 32 KB: one operand of one step
constexpr int kBufs = 5;                        // 160 KB: the whole LDS
constexpr int kLoadsPerOp = kBufBytes / 1024 / (kThreads / kWave);  // 8 x 1 KB per wave
// One tail-split unit's partial tile: 4 waves x 16 (i, j) MFMA blocks x 4 x 64
// lanes of f32x4, stored in register order so every store is 1 KB contiguous.
constexpr int kPartVecsPerWave = 4 * 4 * 4 * kWave;

// Physical 16-byte chunk of logical chunk c (0..7) in the 128-byte LDS row r.
// Two consecutive rows fill one 256-byte span of the 64-bank LDS; XOR with
// (r >> 1) & 7 gives the eight row pairs of any 16 consecutive rows different
// chunk columns, so 16 rows read at one logical chunk hit 16 distinct 16-byte
// bank groups. The map is an involution.
__device__ __forceinline__ uint32_t swz8(int c, int r) {
  return static_cast<uint32_t>(c ^ ((r >> 1) & 7));
}

// Token row (offset in the tile) of lane row lr of token block j of a wave
// with token half wave_t, on 256-row tiles or on the 128-row tiles of
// ffn_tiled_half_kernel (two 32-row blocks per wave); kTileT when the block is
// unused (the fix-up kernels serve both).
__device__ __forceinline__ int tile_row_of_block(bool half, int wave_t, int j, int lr) {
  return half ? (j < 2 ? wave_t * 64 + j * 32 + lr : kTileT) : wave_t * 128 + j * 32 + lr;
}

__device__ __forceinline__ int ring_add(int b, int n) {  // (b + n) % kBufs, 0 <= n < kBufs
  b += n;
  return b >= kBufs ? b - kBufs : b;
}

// A work item or a K-part of a split tail item: its tile, step range and
// partial-tile slot (-1 for a whole item).
struct Work {
  Tile t;
  int kb, ke, unit;
};

__device__ __forceinline__ Work decode_work(const FfnArgs& a, const WorkSplit& ws, int L,
                                            int per_split, int n_t, int nk, int tile_rows) {
  Work w;
  if (L < ws.n_full) {
    w.t = decode_tile(a, L, per_split, n_t, tile_rows);
    w.kb = 0;
    w.ke = nk;
    w.unit = -1;
  } else {
    const int u = L - ws.n_full, len = nk / ws.S;
    w.t = decode_tile(a, ws.n_full + u / ws.S, per_split, n_t, tile_rows);
    w.kb = (u % ws.S) * len;
    w.ke = w.kb + len;
    w.unit = u;
  }
  return w;
}

// Persistent: one workgroup per CU walks work items L = L0, L0 + G, ... (G =
// grid size) of the (split, weight tile, token tile) space. Its steps form one
// continuous stream; two load cursors (weights, tokens) walk it ahead of the
// MFMAs and cross into the next item while the current one is still being
// multiplied, so no workgroup launch or pipeline fill is paid per tile.
// Operand W_s (weights of step s) sits in LDS buffer (2s) % 5, X_s (tokens) in
// (2s + 1) % 5; W_{s+2} goes to the buffer of X_{s-1} and X_{s+2} to that of
// W_s.
//
// Each wave's 128x128 sub-tile is 8x8 blocks of v_mfma_f32_16x16x32 (64
// accumulators of 4 fp32). On random bf16 operands this MFMA does 15 % more
// FLOPs per joule than v_mfma_f32_32x32x16 (a probe with every SIMD busy on
// either: 2.13 against 1.85 PFLOP/s at the power limit), and the kernel is
// power bound (Mixtral shape, 4096 tokens: gate_up 1.64 -> 1.52 ms). A step is
// two 32-k sub-steps of 64 MFMAs per wave:
//   sub-step 0: MFMAs (s, 0); read (s, 1); issue W_{s+2}
//   barrier B_s: at most the 8 W_{s+2} loads in flight (vmcnt(8)), so W_{s+1}
//               and X_{s+1} have landed; step s's buffers are no longer read
//   sub-step 1: MFMAs (s, 1); read (s+1, 0); issue X_{s+2} into the buffer of
//               W_s
// Tokens thus get ~1.5 sub-steps of lead and weights ~3 (a token tile is
// mostly not in L2 when its first CU of an XCD asks for it).
// Operand fragments: lane l reads row (l & 15) of a 16-row block at logical
// chunk 4h + (l >> 4) of the 128-byte row (k 32h + 8 (l >> 4) .. +7); 16 lanes
// of one chunk hit 16 distinct bank groups under swz8. Lane l of output block
// (bi, bj) holds features 4 (l >> 4) + 0..3 of weight block bi and token
// (l & 15) of token block bj.
// c += a * b on v_mfma_f32_16x16x32 for accumulator block n, pinned to
// a[4n .. 4n+3] (acc_regs.h). The compiler holds no accumulator values (with
// compiled MFMAs on 64 f32x4 accumulators it had put results in other
// registers than their accumulators and copied between them).
template <typename T, int n>
__device__ __forceinline__ void mfma16_acc(u32x4 a, u32x4 b) {
  if constexpr (std::is_same<T, bf16>::value)
    accr::mfma_bf16<n>(a, b);
  else
    accr::mfma_f16<n>(a, b);
}

// f(std::integral_constant<int, k>) for k = B .. E-1, expanded at compile
// time (accumulator registers are named by literal strings, so every index
// that reaches them must be a constant).
template <int B, int E, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (B < E) {
    f(std::integral_constant<int, B>{});
    static_for<B + 1, E>(f);
  }
}

typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// Four values rounded to T (bf16 or f16), packed in two dwords.
template <typename T>
__device__ __forceinline__ u32x2 pack4(float a, float b, float c, float d) {
  typedef T T4 __attribute__((ext_vector_type(4)));
  const T4 v = {from_f32<T>(a), from_f32<T>(b), from_f32<T>(c), from_f32<T>(d)};
  return __builtin_bit_cast(u32x2, v);
}

template <typename T, bool kGateUp, bool kRagged>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(1, 1)))
__attribute__((amdgpu_num_vgpr(128)))
void ffn_tiled16_kernel(const FfnArgs a) {
  __shared__ __attribute__((aligned(1024))) uint8_t lds[kBufs * kBufBytes];

  const int tid = threadIdx.x, lane = tid & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int wave_w = wave >> 1, wave_t = wave & 1;

  const int n_t = a.tile_map[0];
  const int per_split = a.n_wtiles * n_t;
  const int n_work = a.splits * per_split;
  const int G = gridDim.x;
  const int nk = a.k_per_split / kSK;
  const WorkSplit ws = work_split(n_work, G, nk, a.part_units);
  const int n_seq = ws.n_full + ws.n_units;
  int Lc = xcd_remap(blockIdx.x, G);
  if (Lc >= n_seq) return;
  // Item sequence of this workgroup: slot s (its place on the XCD) of its
  // XCD's block of n_x consecutive items in every round (items k G .. k G +
  // G - 1). kRagged launches (experts holding few token tiles each) multiply
  // only the token blocks an item's rows reach, so an expert's last-tile
  // items are cheaper than its others; they also take, in the rounds wholly
  // made of full items, slot (s + 13 k) mod n_x instead of s, so that which
  // CUs draw those cheaper items changes from round to round instead of
  // falling on the same CUs every round. Both pay where experts hold few
  // tiles (Phi-3.5 2048 tokens gate_up -4 %, fine-grained 4096 tokens -4 %)
  // and cost where they hold many (Mixtral 4096 tokens +4 %: CUs that drew
  // cheap items run into the next round early and no longer share its
  // weight slabs in L2).
  // A cursor is (item L, round k, rotated slot r); next() gives the next
  // one without a division (it runs at item boundaries of the K loop).
  const int xslot = blockIdx.x >> 3;
  const int n_x = (G >> 3) + ((blockIdx.x & 7) < (G & 7) ? 1 : 0);
  const int xbase = Lc - xslot, rstep = kRagged ? 13 % n_x : 0;
  struct Seq {
    int L, k, r;
  };
  auto next = [&](const Seq& c) {
    if (!kRagged) return Seq{c.L + G, c.k + 1, c.r};
    Seq n{0, c.k + 1, c.r + rstep};
    if (n.r >= n_x) n.r -= n_x;
    n.L = n.k * G + xbase + ((n.k + 1) * G <= ws.n_full ? n.r : xslot);
    return n;
  };

  const int ld = kGateUp ? a.H : a.I;
  const uint32_t pitch = static_cast<uint32_t>(ld * 2);
  auto decode = [&](int L) { return decode_work(a, ws, L, per_split, n_t, nk, kTileT); };
  auto op_row = [&](int q, int ln) { return (wave * kLoadsPerOp + q) * 8 + (ln >> 3); };

  Seq wq{Lc, 0, xslot};
  int wkt = 0, wke = 0;
  __amdgpu_buffer_rsrc_t wsrc;
  uint32_t woff[kLoadsPerOp];
  auto setup_w = [&](const Work& w) {
    const Tile& t = w.t;
    wkt = w.kb;
    wke = w.ke;
    const int ln = opaque(lane);
    wsrc = lds_rsrc(static_cast<const char*>(a.w[t.e]) + static_cast<size_t>(t.split) * a.k_per_split * 2,
                    -1);
#pragma unroll
    for (int q = 0; q < kLoadsPerOp; ++q) {
      const int r = op_row(q, ln);
      const int wr = kGateUp ? (r < kTileW / 2 ? t.wtile * (kTileW / 2) + r
                                               : a.I + t.wtile * (kTileW / 2) + (r - kTileW / 2))
                             : t.wtile * kTileW + r;
      woff[q] = static_cast<uint32_t>(wr) * pitch + swz8(ln & 7, r) * 16;
    }
  };

  Seq xq{Lc, 0, xslot};
  int xkt = 0, xke = 0;
  __amdgpu_buffer_rsrc_t xsrc;
  uint32_t xoff[kLoadsPerOp];
  int grow[kLoadsPerOp];
  auto fetch_rows = [&](const Tile& t) {
    const int ln = opaque(lane);
#pragma unroll
    for (int q = 0; q < kLoadsPerOp; ++q) grow[q] = a.row_src[min(t.row0 + op_row(q, ln), t.row_end - 1)];
  };
  auto setup_x = [&](const Work& w) {
    const Tile& t = w.t;
    xkt = w.kb;
    xke = w.ke;
    const int ln = opaque(lane);
    const size_t kbeg = static_cast<size_t>(t.split) * a.k_per_split;
    // Rows past the group's end load zeros (offsets with bit 31 set).
    if (kGateUp) {
      xsrc = lds_rsrc(static_cast<const char*>(a.x) + kbeg * 2);
#pragma unroll
      for (int q = 0; q < kLoadsPerOp; ++q) {
        const int r = op_row(q, ln);
        const uint32_t pad = t.row0 + r < t.row_end ? 0u : kPadOffset;
        xoff[q] = (static_cast<uint32_t>(grow[q]) * pitch + swz8(ln & 7, r) * 16) | pad;
      }
    } else {
      xsrc = lds_rsrc(static_cast<const char*>(a.x) +
                      (static_cast<size_t>(t.row0) * ld + kbeg) * 2);
#pragma unroll
      for (int q = 0; q < kLoadsPerOp; ++q) {
        const int r = op_row(q, ln);
        const uint32_t pad = t.row0 + r < t.row_end ? 0u : kPadOffset;
        xoff[q] = (static_cast<uint32_t>(r) * pitch + swz8(ln & 7, r) * 16) | pad;
      }
    }
  };
  auto prefetch_next_rows = [&]() {
    if (kGateUp) {
      const int n = next(xq).L;
      fetch_rows(decode(n < n_seq ? n : xq.L).t);
    }
  };
  auto advance_w = [&]() {
    if (++wkt < wke) return;
    const Seq n = next(wq);
    if (n.L < n_seq) {
      wq = n;
      setup_w(decode(wq.L));
    } else {
      wkt = wke - 1;
    }
  };
  auto advance_x = [&]() {
    if (++xkt < xke) return;
    const Seq n = next(xq);
    if (n.L < n_seq) {
      xq = n;
      setup_x(decode(xq.L));
      prefetch_next_rows();
    } else {
      xkt = xke - 1;
    }
  };
  auto issue_w = [&](int b, int q) {
    dma16_rsrc(wsrc, woff[q], wkt * kSRowBytes, lds + b * kBufBytes + (wave * kLoadsPerOp + q) * 1024);
  };
  auto issue_x = [&](int b, int q) {
    dma16_rsrc(xsrc, xoff[q], xkt * kSRowBytes, lds + b * kBufBytes + (wave * kLoadsPerOp + q) * 1024);
  };

  // MFMA operand rows of this wave: weight blocks bi (gate_up: 0-3 gate rows
  // 64 wave_w + 16 bi, 4-7 the matching up rows 128 + ..; down 128 wave_w +
  // 16 bi), token blocks 16 (2 bj + wave_t): the two token waves interleave
  // 16-row blocks, so the first 32 J rows of a tile are token blocks 0 .. J-1
  // of both. A lane reads row (l & 15) of a block at logical chunk 4 h +
  // (l >> 4); a block's place in the buffer is an immediate offset of the
  // read, so one base address per operand and k-half serves all 8 blocks.
  const int lr = lane & 15, kq = lane >> 4;
  const uint32_t lds0 =
      static_cast<uint32_t>(reinterpret_cast<size_t>((const __attribute__((address_space(3))) uint8_t*)lds));
  uint32_t abase[2], bbase[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    // Block rows start at multiples of 16, so the swizzle bits are lr's.
    const uint32_t coff = swz8(4 * h + kq, lr) << 4;
    abase[h] = lds0 + ((kGateUp ? wave_w * 64 : wave_w * 128) + lr) * kSRowBytes + coff;
    bbase[h] = lds0 + (wave_t * 16 + lr) * kSRowBytes + coff;
  }
  // Byte offsets of weight block i and token block j from those bases.
  auto a_off = [](auto ic) {
    constexpr int i = decltype(ic)::value;
    return std::integral_constant<int, (16 * i + (kGateUp && i >= 4 ? 64 : 0)) * kSRowBytes>{};
  };
  auto b_off = [](auto jc) { return std::integral_constant<int, 32 * decltype(jc)::value * kSRowBytes>{}; };

  // Accumulator block (i, j) is AGPR block 8 i + j (a[4 (8 i + j) ..]); the
  // indices are integral constants.
  auto acc_at = [](auto i, auto j, auto r) {
    return accr::get<4 * (8 * decltype(i)::value + decltype(j)::value) + decltype(r)::value>();
  };
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  using I2 = std::integral_constant<int, 2>;
  using I3 = std::integral_constant<int, 3>;
  // The MFMAs are assembly, out of the compiler's hazard checks: an MFMA
  // reading as accumulator an AGPR that a VALU op wrote needs 2 wait states
  // (after zeroing), and a read of an MFMA result needs up to 11 for these
  // 4-pass MFMAs (before the epilogue); mfma_nops() gives 24.
  auto mfma_nops = []() {
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("s_nop 7\n s_nop 7\n s_nop 7");
    __builtin_amdgcn_sched_barrier(0);
  };
  auto zero_acc = [&]() {
    accr::zero_all();
    mfma_nops();
  };
  // Operand fragments live in fixed VGPRs above the compiler's budget
  // (acc_regs.h): set s holds weight block i at v[128 + 32 s + 4 i ..] and
  // token block j at v[192 + 32 s + 4 j ..]. Reads and MFMAs are assembly,
  // so the compiler keeps only addresses, and the K loop can exist in one copy
  // per token-block count J without register pressure.
  auto read_a = [&](auto sc, auto ic, uint32_t base) {
    accr::Frag<128 + 32 * decltype(sc)::value + 4 * decltype(ic)::value>::template read<
        decltype(a_off(ic))::value>(base);
  };
  auto read_b = [&](auto sc, auto jc, uint32_t base) {
    accr::Frag<192 + 32 * decltype(sc)::value + 4 * decltype(jc)::value>::template read<
        decltype(b_off(jc))::value>(base);
  };
  auto read_frags = [&](int bw, int bx, int h, auto sc) {
    const uint32_t av = abase[h] + bw * kBufBytes, bv = bbase[h] + bx * kBufBytes;
    static_for<0, 8>([&](auto b) {
      read_a(sc, b, av);
      read_b(sc, b, bv);
    });
  };

  // One sub-step on fragment set S: wait for its operands, then the 8 J
  // MFMAs of weight blocks 0-7 x token blocks 0 .. J-1 (a tile of n rows
  // needs J = ceil(n / 32)), with the next sub-step's 16 operand reads (into
  // set 1 - S) and 8 loads spread over them: at J = 8 reads after MFMAs 1, 4,
  // .., 46 and loads after MFMAs 2, 5, .., 23, the last 16 MFMAs giving the
  // last reads time to land; at smaller J the same pattern compressed. All 8
  // token blocks are read whatever J is, so the reads do not depend on the
  // next item's J. The MFMAs are volatile assembly, so this program order is
  // the issue order (the reads and loads cannot move across them). Weight
  // block i's J MFMAs run token blocks up for even i and down for odd i, so
  // consecutive MFMAs share one operand also where i changes: one operand
  // change per MFMA instead of two at each of the 7 row changes (Mixtral
  // shape, 4096 tokens: gate_up 1469 -> 1459 us over three interleaved pairs,
  // outputs bit-identical; each accumulator still sums k in order).
  auto sub = [&](auto sc, int bw, int bx, int h, auto issue, auto jc) {
    constexpr int S = decltype(sc)::value, J = decltype(jc)::value, M = 8 * J;
    using NS = std::integral_constant<int, 1 - S>;
    wait_lgkm0();
    const uint32_t av = abase[h] + bw * kBufBytes, bv = bbase[h] + bx * kBufBytes;
    static_for<0, M>([&](auto mc) {
      constexpr int m = decltype(mc)::value, i = m / J, j = (i & 1) ? J - 1 - m % J : m % J;
      if constexpr (std::is_same<T, bf16>::value)
        accr::mma_bf16<S, i, j>();
      else
        accr::mma_f16<S, i, j>();
      static_for<0, 16>([&](auto rc) {  // reads A0 B0 A1 B1 ..
        constexpr int r = decltype(rc)::value;
        if constexpr ((3 * r + 1) * M / 64 == m) {
          if constexpr (r & 1)
            read_b(NS{}, std::integral_constant<int, (r >> 1)>{}, bv);
          else
            read_a(NS{}, std::integral_constant<int, (r >> 1)>{}, av);
        }
      });
      static_for<0, kLoadsPerOp>([&](auto qc) {
        if constexpr ((3 * decltype(qc)::value + 2) * M / 64 == m) issue(decltype(qc)::value);
      });
    });
  };

  // Prologue: W_0, X_0, W_1 and X_1 (the loads sub-step 1 of step -1 would
  // issue), then wait for W_0 and X_0 and read (0, 0).
  {
    const Work w0 = decode(Lc);
    if (kGateUp) fetch_rows(w0.t);
    setup_w(w0);
    setup_x(w0);
    prefetch_next_rows();
  }
#pragma unroll
  for (int q = 0; q < kLoadsPerOp; ++q) issue_w(0, q);
  advance_w();
#pragma unroll
  for (int q = 0; q < kLoadsPerOp; ++q) issue_x(1, q);
  advance_x();
#pragma unroll
  for (int q = 0; q < kLoadsPerOp; ++q) issue_w(2, q);
  advance_w();
#pragma unroll
  for (int q = 0; q < kLoadsPerOp; ++q) issue_x(3, q);
  advance_x();
  dma_barrier<2 * kLoadsPerOp>();  // W_0 and X_0 landed

  zero_acc();
  read_frags(0, 1, 0, std::integral_constant<int, 0>{});

  int bw = 0;  // buffer of W_s (X_s is in the next one)
  Seq cq{Lc, 0, xslot};
  Work cw = decode(Lc);
  while (true) {
    const Tile& ct = cw.t;
    using S0 = std::integral_constant<int, 0>;
    using S1 = std::integral_constant<int, 1>;
    auto kloop = [&](auto jc) {
      for (int kt = cw.kb; kt < cw.ke; ++kt) {
        const int bx = ring_add(bw, 1);
        const int nbw = ring_add(bw, 2), nbx = ring_add(bw, 3);  // step s+1
        const int bw2 = ring_add(bw, 4);                          // W_{s+2}
        // W_{s+2} (its buffer held X_{s-1}, freed by B_{s-1}).
        sub(S0{}, bw, bx, 1, [&](int i) { issue_w(bw2, i); }, jc);
        advance_w();
        // W_{s+1} and X_{s+1} landed (only W_{s+2} may be in flight) and every
        // wave has read its last operands of step s.
        wait_lgkm0();
        dma_barrier<kLoadsPerOp>();
        // X_{s+2} into the buffer of W_s.
        sub(S1{}, nbw, nbx, 0, [&](int i) { issue_x(bw, i); }, jc);
        advance_x();
        bw = nbw;
      }
    };
    // Token blocks J per wave (32 J tile rows): kRagged, the blocks the item's
    // rows reach; otherwise those of the expert's tile height, the same for
    // all of its items (an expert's items in one XCD round then take equally
    // long). Rows past the item's end are zero-filled in the LDS; blocks past
    // J are not multiplied. J = 1 and 3 run as 2 and 4 (fewer K-loop copies).
    switch (min(8, ((kRagged ? ct.row_end - ct.row0 : ct.height) + 31) >> 5)) {
      case 1:
      case 2: kloop(std::integral_constant<int, 2>{}); break;
      case 3:
      case 4: kloop(std::integral_constant<int, 4>{}); break;
      case 5: kloop(std::integral_constant<int, 5>{}); break;
      case 6: kloop(std::integral_constant<int, 6>{}); break;
      case 7: kloop(std::integral_constant<int, 7>{}); break;
      default: kloop(std::integral_constant<int, 8>{}); break;
    }

    mfma_nops();
    const int eln = opaque(lane), elr = eln & 15, ekq = eln >> 4;
    if (cw.unit >= 0) {
      // K-part of a split tail item: raw fp32 accumulators to its partial slot,
      // block by block (each store 1 KB contiguous).
      f32x4* pp = reinterpret_cast<f32x4*>(a.part) +
                  static_cast<size_t>(cw.unit * 4 + wave) * kPartVecsPerWave + eln;
      static_for<0, 8>([&](auto i) {
        static_for<0, 8>([&](auto j) {
          pp[(i * 8 + j) * kWave] = f32x4{acc_at(i, j, I0{}), acc_at(i, j, I1{}), acc_at(i, j, I2{}),
                                          acc_at(i, j, I3{})};
        });
      });
      zero_acc();
    } else if (kGateUp) {
      T* inter = static_cast<T*>(a.out);
      auto epilogue = [&](auto silu) {
        static_for<0, 8>([&](auto j) {
          const int prow = ct.row0 + (2 * j + wave_t) * 16 + elr;
          if (prow < ct.row_end) {
            static_for<0, 4>([&](auto i) {
              using IU = std::integral_constant<int, decltype(i)::value + 4>;
              const int col = ct.wtile * (kTileW / 2) + wave_w * 64 + i * 16 + 4 * ekq;
              float v[4];
              static_for<0, 4>([&](auto r) {
                v[decltype(r)::value] =
                    gate_act_16<decltype(silu)::value>(a.act, acc_at(i, j, r)) * acc_at(IU{}, j, r);
              });
              store4<T>(inter + static_cast<size_t>(prow) * a.I + col, v[0], v[1], v[2], v[3]);
            });
          }
          static_for<0, 8>([&](auto i) { accr::zero_block<8 * decltype(i)::value + decltype(j)::value>(); });
          __builtin_amdgcn_sched_barrier(0);
        });
      };
      if (a.act == MOE355_ACT_SILU)
        epilogue(std::true_type{});
      else
        epilogue(std::false_type{});
      mfma_nops();
    } else {
      // y: the 4 lanes holding one token row's features of a block (lanes
      // r, r + 16, r + 32, r + 48) are far apart, so a store straight from
      // the MFMA layout reaches memory as 64 separate 8-byte pieces. A lane
      // permutation first (lane 4 r + q takes lane r + 16 q's values) puts each
      // row's 32 bytes in 4 consecutive lanes; the stores then coalesce into
      // 16 row pieces (down at 1408-wide K: epilogue 11.7 -> 6.8 k cycles).
      const int pr = eln >> 2, pq = eln & 3;
      const int psrc = (pr + 16 * pq) << 2;
      auto perm = [&](uint32_t v) {
        return static_cast<uint32_t>(__builtin_amdgcn_ds_bpermute(psrc, static_cast<int>(v)));
      };
      auto store_y = [&](auto* y) {
        using O = typename std::remove_pointer<decltype(y)>::type;
        static_for<0, 8>([&](auto j) {
          const int prow = ct.row0 + (2 * j + wave_t) * 16 + pr;
          O* yr = y + static_cast<size_t>(prow) * a.H + (ct.wtile * kTileW + wave_w * 128 + 4 * pq);
          if constexpr (sizeof(O) == 4) {
            u32x4 q[8];
            static_for<0, 8>([&](auto i) {
              static_for<0, 4>([&](auto r) {
                q[i][decltype(r)::value] = perm(__builtin_bit_cast(uint32_t, acc_at(i, j, r)));
              });
            });
            if (prow < ct.row_end) {
#pragma unroll
              for (int i = 0; i < 8; ++i) *reinterpret_cast<u32x4*>(yr + i * 16) = q[i];
            }
          } else {
            u32x2 q[8];
            static_for<0, 8>([&](auto i) {
              const u32x2 pk = pack4<O>(acc_at(i, j, I0{}), acc_at(i, j, I1{}), acc_at(i, j, I2{}),
                                        acc_at(i, j, I3{}));
              q[i] = u32x2{perm(pk[0]), perm(pk[1])};
            });
            if (prow < ct.row_end) {
#pragma unroll
              for (int i = 0; i < 8; ++i) *reinterpret_cast<u32x2*>(yr + i * 16) = q[i];
            }
          }
          static_for<0, 8>([&](auto i) { accr::zero_block<8 * decltype(i)::value + decltype(j)::value>(); });
          __builtin_amdgcn_sched_barrier(0);
        });
      };
      if (a.y16)
        store_y(static_cast<T*>(a.out));
      else
        store_y(static_cast<float*>(a.out) + static_cast<size_t>(ct.split) * a.R * a.H);
      mfma_nops();
    }
    cq = next(cq);
    if (cq.L >= n_seq) break;
    cw = decode(cq.L);
  }
  wait_vmcnt<0>();
}

// 128-row token tiles (groups of about 128 rows or fewer). Few tokens meet
// each weight slab, so a step carries a quarter of a full tile's MFMA work
// (~256 cycles per sub-step) and the loads' latency shows. Token rows are
// mostly not in L2 (the weight stream evicts them) and come from the
// Infinity Cache, ~1 us away: issued one step ahead, as in the full-tile
// pipeline, they arrive after the barrier that waits for them. And in one
// wave's counter loads retire in order, so waiting for tokens also waits for
// every weight load issued before them.
//
// Here waves 0-1 issue all weight loads and waves 2-3 all token loads (every
// wave still multiplies), so each wave's counter holds one kind of load only.
// The LDS holds a ring of three 32 KB weight buffers and four 16 KB token
// buffers (128 rows, compact), 160 KB in all: weights are issued two steps
// ahead of their use (a plain stream reaches ~6.3 TB/s with 32 KB in flight
// per CU), tokens three.
//   step s, weight buffer s % 3, token buffer s % 4; sub-step j (16 k each):
//   sub-step 0: MFMAs (s, 0), read (s, 1); W_{s+2} loads 4-7, X_{s+3} loads 4-7
//   sub-step 1: MFMAs (s, 1), read (s, 2); W_{s+2} loads 8-11
//   sub-step 2: MFMAs (s, 2), read (s, 3); W_{s+2} loads 12-15
//   barrier B_s: weight waves wait until at most their 16 loads of W_{s+2} are
//                in flight (so W_{s+1} has landed), token waves until at most
//                their 16 of X_{s+2} and X_{s+3} (so X_{s+1} has).
//   sub-step 3: MFMAs (s, 3), read (s+1, 0); W_{s+3} loads 0-3 into the buffer
//               of W_s, X_{s+4} loads 0-3 into the buffer of X_s (both freed
//               by B_s).
// Each wave multiplies its 128 weight rows against its two 32-row token
// blocks (token half wave_t: tile rows 64 wave_t ..); the lane layout of the
// accumulators, the epilogue and the K-split partial tiles are those of the
// full-tile kernel with token blocks 0-1.
constexpr int kHalfRows = kTileT / 2;
constexpr int kXBufBytes = kHalfRows * kSRowBytes;        // 16 KB
constexpr int kWBufs = 3, kXBufs = 4;                      // 3 x 32 KB + 4 x 16 KB = 160 KB
constexpr int kWLoadsPerWave = kBufBytes / 1024 / 2;       // 16 x 1 KB per weight wave
constexpr int kXLoadsPerWave = kXBufBytes / 1024 / 2;      // 8 x 1 KB per token wave
static_assert(kWBufs * kBufBytes + kXBufs * kXBufBytes == kBufs * kBufBytes, "LDS budget");

template <typename T, bool kGateUp, bool kWeightWave>
__device__ __forceinline__ void half_tile_waves(const FfnArgs& a, uint8_t* lds, int wave,
                                                int lane, int Lc) {
  const int wave_w = wave >> 1, wave_t = wave & 1;
  const int lw = wave & 1;  // this wave's share of its kind of load
  const int n_t = a.tile_map[0];
  const int per_split = a.n_wtiles * n_t;
  const int G = gridDim.x;
  const int nk = a.k_per_split / kSK;
  const WorkSplit ws = work_split(a.splits * per_split, G, nk, a.part_units);
  const int n_seq = ws.n_full + ws.n_units;
  const int ld = kGateUp ? a.H : a.I;
  const uint32_t pitch = static_cast<uint32_t>(ld * 2);
  auto decode = [&](int L) { return decode_work(a, ws, L, per_split, n_t, nk, kHalfRows); };
  auto wbuf = [&](int b) { return lds + b * kBufBytes; };
  auto xbuf = [&](int b) { return lds + kWBufs * kBufBytes + b * kXBufBytes; };

  // Weight cursor (weight waves): rows (16 lw + q) * 8 + lane / 8, q < 16.
  int wL = Lc, wkt = 0, wke = 0;
  __amdgpu_buffer_rsrc_t wsrc;
  uint32_t woff[kWLoadsPerWave];
  auto w_row = [&](int q, int ln) { return (lw * kWLoadsPerWave + q) * 8 + (ln >> 3); };
  auto setup_w = [&](const Work& w) {
    const Tile& t = w.t;
    wkt = w.kb;
    wke = w.ke;
    const int ln = opaque(lane);
    wsrc = lds_rsrc(static_cast<const char*>(a.w[t.e]) + static_cast<size_t>(t.split) * a.k_per_split * 2,
                    -1);
#pragma unroll
    for (int q = 0; q < kWLoadsPerWave; ++q) {
      const int r = w_row(q, ln);
      const int wr = kGateUp ? (r < kTileW / 2 ? t.wtile * (kTileW / 2) + r
                                               : a.I + t.wtile * (kTileW / 2) + (r - kTileW / 2))
                             : t.wtile * kTileW + r;
      woff[q] = static_cast<uint32_t>(wr) * pitch + swz8(ln & 7, r) * 16;
    }
  };
  auto advance_w = [&]() {
    if (++wkt < wke) return;
    if (wL + G < n_seq) {
      wL += G;
      setup_w(decode(wL));
    } else {
      wkt = wke - 1;
    }
  };
  auto issue_w = [&](int b, int q0, int n) {
    uint8_t* dst = wbuf(b) + lw * kWLoadsPerWave * 1024;
#pragma unroll
    for (int q = q0; q < q0 + n; ++q) dma16_rsrc(wsrc, woff[q], wkt * kSRowBytes, dst + q * 1024);
  };

  // Token cursor (token waves): tile rows (8 lw + q) * 8 + lane / 8, q < 8;
  // gate_up rows come through row_src, fetched one item ahead.
  int xL = Lc, xkt = 0, xke = 0;
  __amdgpu_buffer_rsrc_t xsrc;
  uint32_t xoff[kXLoadsPerWave];
  int grow[kXLoadsPerWave];
  auto x_row = [&](int q, int ln) { return (lw * kXLoadsPerWave + q) * 8 + (ln >> 3); };
  auto fetch_rows = [&](const Tile& t) {
    const int ln = opaque(lane);
#pragma unroll
    for (int q = 0; q < kXLoadsPerWave; ++q)
      grow[q] = a.row_src[min(t.row0 + x_row(q, ln), t.row_end - 1)];
  };
  auto setup_x = [&](const Work& w) {
    const Tile& t = w.t;
    xkt = w.kb;
    xke = w.ke;
    const int ln = opaque(lane);
    const size_t kbeg = static_cast<size_t>(t.split) * a.k_per_split;
    // Rows past the group's end load zeros (offsets with bit 31 set, as in the
    // full-tile kernel).
    if (kGateUp) {
      xsrc = lds_rsrc(static_cast<const char*>(a.x) + kbeg * 2);
#pragma unroll
      for (int q = 0; q < kXLoadsPerWave; ++q) {
        const int r = x_row(q, ln);
        const uint32_t pad = t.row0 + r < t.row_end ? 0u : kPadOffset;
        xoff[q] = (static_cast<uint32_t>(grow[q]) * pitch + swz8(ln & 7, r) * 16) | pad;
      }
    } else {
      xsrc = lds_rsrc(static_cast<const char*>(a.x) +
                      (static_cast<size_t>(t.row0) * ld + kbeg) * 2);
#pragma unroll
      for (int q = 0; q < kXLoadsPerWave; ++q) {
        const int r = x_row(q, ln);
        const uint32_t pad = t.row0 + r < t.row_end ? 0u : kPadOffset;
        xoff[q] = (static_cast<uint32_t>(r) * pitch + swz8(ln & 7, r) * 16) | pad;
      }
    }
  };
  auto prefetch_next_rows = [&]() {
    if (kGateUp) fetch_rows(decode(xL + G < n_seq ? xL + G : xL).t);
  };
  auto advance_x = [&]() {
    if (++xkt < xke) return;
    if (xL + G < n_seq) {
      xL += G;
      setup_x(decode(xL));
      prefetch_next_rows();
    } else {
      xkt = xke - 1;
    }
  };
  auto issue_x = [&](int b, int q0, int n) {
    uint8_t* dst = xbuf(b) + lw * kXLoadsPerWave * 1024;
#pragma unroll
    for (int q = q0; q < q0 + n; ++q) dma16_rsrc(xsrc, xoff[q], xkt * kSRowBytes, dst + q * 1024);
  };

  // MFMA operand rows of this wave: weight blocks as in the full-tile kernel,
  // token blocks 64 wave_t + 32 b (b < 2) of the compact token buffer.
  const int lr = lane & 31, kh = lane >> 5;
  uint32_t arow[4], brow[2];
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    const int rb = kGateUp ? (b < 2 ? wave_w * 64 + b * 32 : kTileW / 2 + wave_w * 64 + (b - 2) * 32)
                           : wave_w * 128 + b * 32;
    arow[b] = (rb + lr) * kSRowBytes;
  }
#pragma unroll
  for (int b = 0; b < 2; ++b) brow[b] = (wave_t * 64 + b * 32 + lr) * kSRowBytes;
  uint32_t coff[kSK / 16];
#pragma unroll
  for (int j = 0; j < kSK / 16; ++j) coff[j] = swz8(2 * j + kh, lr) << 4;

  f32x16 acc[4][2];
  auto acc_read = [](float x) {
    float r;
    asm volatile("v_accvgpr_read_b32 %0, %1" : "=v"(r) : "a"(x));
    return r;
  };
  auto zero_acc = [&]() {
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) acc[i][j] = f32x16{};
  };
  auto read_frags = [&](int bw, int bx, int j, u32x4* af, u32x4* bf) {
    const uint8_t* sw = wbuf(bw);
    const uint8_t* sx = xbuf(bx);
#pragma unroll
    for (int b = 0; b < 4; ++b) af[b] = *reinterpret_cast<const u32x4*>(sw + arow[b] + coff[j]);
#pragma unroll
    for (int b = 0; b < 2; ++b) bf[b] = *reinterpret_cast<const u32x4*>(sx + brow[b] + coff[j]);
  };

  // One sub-step: wait for its operands, 8 MFMAs; the next sub-step's 6
  // operand reads and NL loads spread over them.
  auto sub = [&](const u32x4* af, const u32x4* bf, int bw, int bx, int j, u32x4* na, u32x4* nb,
                 auto issue, auto nl) {
    constexpr int NL = decltype(nl)::value;
    wait_lgkm0();
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int jj = 0; jj < 2; ++jj) acc[i][jj] = Mfma32<T>::mma(af[i], bf[jj], acc[i][jj]);
    const uint8_t* sw = wbuf(bw);
    const uint8_t* sx = xbuf(bx);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      na[i] = *reinterpret_cast<const u32x4*>(sw + arow[i] + coff[j]);
      if (i < NL) issue(i);
      if (i < 2) nb[i] = *reinterpret_cast<const u32x4*>(sx + brow[i] + coff[j]);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);    // MFMA
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);    // LDS read
      if (i < NL) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // global -> LDS load
      if (i < 2) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
  };
  using L4 = std::integral_constant<int, 4>;
  using L0 = std::integral_constant<int, 0>;
  auto none = [](int) {};

  // Prologue: weight waves W_0, W_1 and loads 0-3 of W_2 (wait for W_0);
  // token waves X_0, X_1, X_2 and loads 0-3 of X_3 (wait for X_0).
  {
    const Work w0 = decode(Lc);
    if (kWeightWave) {
      setup_w(w0);
      issue_w(0, 0, kWLoadsPerWave);
      advance_w();
      issue_w(1, 0, kWLoadsPerWave);
      advance_w();
      issue_w(2, 0, 4);
      wait_vmcnt<kWLoadsPerWave + 4>();
    } else {
      if (kGateUp) fetch_rows(w0.t);
      setup_x(w0);
      prefetch_next_rows();
      issue_x(0, 0, kXLoadsPerWave);
      advance_x();
      issue_x(1, 0, kXLoadsPerWave);
      advance_x();
      issue_x(2, 0, kXLoadsPerWave);
      advance_x();
      issue_x(3, 0, 4);
      wait_vmcnt<2 * kXLoadsPerWave + 4>();
    }
  }
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_barrier();
  __atomic_signal_fence(__ATOMIC_SEQ_CST);

  zero_acc();
  u32x4 fa[2][4], fb[2][2];
  read_frags(0, 0, 0, fa[0], fb[0]);

  int bw = 0, bx = 0;  // buffers of W_s and X_s
  Work cw = decode(Lc);
  while (true) {
    const Tile& ct = cw.t;
    for (int kt = cw.kb; kt < cw.ke; ++kt) {
      const int nbw = bw == kWBufs - 1 ? 0 : bw + 1, nbx = (bx + 1) & (kXBufs - 1);  // step s+1
      const int bw2 = nbw == kWBufs - 1 ? 0 : nbw + 1;                             // W_{s+2}
      const int bx3 = (bx + 3) & (kXBufs - 1);                                     // X_{s+3}
      if (kWeightWave) {
        sub(fa[0], fb[0], bw, bx, 1, fa[1], fb[1], [&](int i) { issue_w(bw2, 4 + i, 1); }, L4{});
        sub(fa[1], fb[1], bw, bx, 2, fa[0], fb[0], [&](int i) { issue_w(bw2, 8 + i, 1); }, L4{});
        sub(fa[0], fb[0], bw, bx, 3, fa[1], fb[1], [&](int i) { issue_w(bw2, 12 + i, 1); }, L4{});
        advance_w();
        wait_lgkm0();
        wait_vmcnt<kWLoadsPerWave>();
      } else {
        sub(fa[0], fb[0], bw, bx, 1, fa[1], fb[1], [&](int i) { issue_x(bx3, 4 + i, 1); }, L4{});
        advance_x();
        sub(fa[1], fb[1], bw, bx, 2, fa[0], fb[0], none, L0{});
        sub(fa[0], fb[0], bw, bx, 3, fa[1], fb[1], none, L0{});
        wait_lgkm0();
        wait_vmcnt<2 * kXLoadsPerWave>();
      }
      __atomic_signal_fence(__ATOMIC_SEQ_CST);
      __builtin_amdgcn_s_barrier();
      __atomic_signal_fence(__ATOMIC_SEQ_CST);
      if (kWeightWave)
        sub(fa[1], fb[1], nbw, nbx, 0, fa[0], fb[0], [&](int i) { issue_w(bw, i, 1); }, L4{});
      else
        sub(fa[1], fb[1], nbw, nbx, 0, fa[0], fb[0], [&](int i) { issue_x(bx, i, 1); }, L4{});
      bw = nbw;
      bx = nbx;
    }

    // Epilogue, as the full-tile kernel's for token blocks 0-1.
    const int eln = opaque(lane), elr = eln & 31, ekh = eln >> 5;
    if (cw.unit >= 0) {
      f32x4* pp = reinterpret_cast<f32x4*>(a.part) +
                  static_cast<size_t>(cw.unit * 4 + wave) * kPartVecsPerWave + eln;
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
          for (int q = 0; q < 4; ++q)
            pp[((i * 4 + j) * 4 + q) * kWave] =
                f32x4{acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2],
                      acc[i][j][4 * q + 3]};
      zero_acc();
    } else if (kGateUp) {
      T* inter = static_cast<T*>(a.out);
      auto epilogue = [&](auto silu) {
#pragma unroll
        for (int b = 0; b < 2; ++b) {
#pragma unroll
          for (int j = 0; j < 2; ++j) {
            const int prow = ct.row0 + wave_t * 64 + j * 32 + elr;
            if (prow < ct.row_end) {
#pragma unroll
              for (int q = 0; q < 4; ++q) {
                const int col = ct.wtile * (kTileW / 2) + wave_w * 64 + b * 32 + 8 * q + 4 * ekh;
                float v[4];
#pragma unroll
                for (int r = 0; r < 4; ++r)
                  v[r] = gate_act_16<decltype(silu)::value>(a.act, acc_read(acc[b][j][4 * q + r])) *
                         acc_read(acc[b + 2][j][4 * q + r]);
                store4<T>(inter + static_cast<size_t>(prow) * a.I + col, v[0], v[1], v[2], v[3]);
              }
            }
            acc[b][j] = f32x16{};
            acc[b + 2][j] = f32x16{};
            __builtin_amdgcn_sched_barrier(0);
          }
        }
      };
      if (a.act == MOE355_ACT_SILU)
        epilogue(std::true_type{});
      else
        epilogue(std::false_type{});
    } else {
      T* y16 = static_cast<T*>(a.out);
      float* y32 = static_cast<float*>(a.out) + static_cast<size_t>(ct.split) * a.R * a.H;
#pragma unroll
      for (int b = 0; b < 4; ++b) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const int prow = ct.row0 + wave_t * 64 + j * 32 + elr;
          if (prow < ct.row_end) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              const int h = ct.wtile * kTileW + wave_w * 128 + b * 32 + 8 * q + 4 * ekh;
              const size_t o = static_cast<size_t>(prow) * a.H + h;
              const float v0 = acc_read(acc[b][j][4 * q]), v1 = acc_read(acc[b][j][4 * q + 1]);
              const float v2 = acc_read(acc[b][j][4 * q + 2]), v3 = acc_read(acc[b][j][4 * q + 3]);
              if (a.y16)
                store4<T>(y16 + o, v0, v1, v2, v3);
              else
                store4<float>(y32 + o, v0, v1, v2, v3);
            }
          }
          acc[b][j] = f32x16{};
          __builtin_amdgcn_sched_barrier(0);
        }
      }
    }
    Lc += G;
    if (Lc >= n_seq) break;
    cw = decode(Lc);
  }
  wait_vmcnt<0>();
}

template <typename T, bool kGateUp>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(1, 1)))
void ffn_tiled_half_kernel(const FfnArgs a) {
  __shared__ __attribute__((aligned(1024))) uint8_t lds[kBufs * kBufBytes];
  const int tid = threadIdx.x, lane = tid & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int n_t = a.tile_map[0];
  const int n_work = a.splits * a.n_wtiles * n_t;
  const WorkSplit ws = work_split(n_work, gridDim.x, a.k_per_split / kSK, a.part_units);
  const int Lc = xcd_remap(blockIdx.x, gridDim.x);
  if (Lc >= ws.n_full + ws.n_units) return;
  if (wave < 2)
    half_tile_waves<T, kGateUp, true>(a, lds, wave, lane, Lc);
  else
    half_tile_waves<T, kGateUp, false>(a, lds, wave, lane, Lc);
}

// Sums the S partial tiles of each split tail item of the tiled gate_up and
// writes act(gate) * up to inter, with the epilogue's lane mapping. Task
// (item, b, j) covers gate block b and up block b + 2 against token block j of
// every wave: 16 KB read per part, 4 KB of inter written at most.
template <typename T>
__global__ __launch_bounds__(kThreads) void gate_up_tail_fixup(const FfnArgs a) {
  const int n_t = a.tile_map[0];
  const int per_split = a.n_wtiles * n_t;
  const int nk = a.k_per_split / kSK;
  const WorkSplit ws = work_split(a.splits * per_split, a.grid, nk, a.part_units);
  const int tasks = ws.n_units / ws.S * 8;
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave;
  const int wave_w = wave >> 1, wave_t = wave & 1, lr = lane & 31, kh = lane >> 5;
  T* inter = static_cast<T*>(a.out);
  for (int task = blockIdx.x; task < tasks; task += gridDim.x) {
    const int it = task >> 3, b = (task >> 2) & 1, j = task & 3;
    const Tile t = decode_tile(a, ws.n_full + it, per_split, n_t, a.tile_rows);
    const int prow = t.row0 + tile_row_of_block(a.tile_rows < kTileT, wave_t, j, lr);
    if (prow >= t.row_end) continue;
    f32x4 g[4] = {}, u[4] = {};
    for (int p = 0; p < ws.S; ++p) {
      const f32x4* pp = reinterpret_cast<const f32x4*>(a.part) +
                        static_cast<size_t>((it * ws.S + p) * 4 + wave) * kPartVecsPerWave + lane;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        g[q] += pp[((b * 4 + j) * 4 + q) * kWave];
        u[q] += pp[(((b + 2) * 4 + j) * 4 + q) * kWave];
      }
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int col = t.wtile * (kTileW / 2) + wave_w * 64 + b * 32 + 8 * q + 4 * kh;
      store4<T>(inter + static_cast<size_t>(prow) * a.I + col, gate_act_fast(a.act, g[q][0]) * u[q][0],
                gate_act_fast(a.act, g[q][1]) * u[q][1], gate_act_fast(a.act, g[q][2]) * u[q][2],
                gate_act_fast(a.act, g[q][3]) * u[q][3]);
    }
  }
}

// Sums the S partial tiles of each split tail item of the tiled down
// projection into the item's y plane (its K-split; Y = the layer dtype when
// y16), with the epilogue's lane mapping. Task (item, b, j) covers weight
// block b against token block j of every wave: 16 KB read per part, 16 KB of
// y written at most.
template <typename Y>
__global__ __launch_bounds__(kThreads) void down_tail_fixup(const FfnArgs a) {
  const int n_t = a.tile_map[0];
  const int per_split = a.n_wtiles * n_t;
  const int nk = a.k_per_split / kSK;
  const WorkSplit ws = work_split(a.splits * per_split, a.grid, nk, a.part_units);
  const int tasks = ws.n_units / ws.S * 16;
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave;
  const int wave_w = wave >> 1, wave_t = wave & 1, lr = lane & 31, kh = lane >> 5;
  for (int task = blockIdx.x; task < tasks; task += gridDim.x) {
    const int it = task >> 4, b = (task >> 2) & 3, j = task & 3;
    const Tile t = decode_tile(a, ws.n_full + it, per_split, n_t, a.tile_rows);
    const int prow = t.row0 + tile_row_of_block(a.tile_rows < kTileT, wave_t, j, lr);
    if (prow >= t.row_end) continue;
    f32x4 v[4] = {};
    for (int p = 0; p < ws.S; ++p) {
      const f32x4* pp = reinterpret_cast<const f32x4*>(a.part) +
                        static_cast<size_t>((it * ws.S + p) * 4 + wave) * kPartVecsPerWave + lane;
#pragma unroll
      for (int q = 0; q < 4; ++q) v[q] += pp[((b * 4 + j) * 4 + q) * kWave];
    }
    Y* y = static_cast<Y*>(a.out) + static_cast<size_t>(t.split) * a.R * a.H;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int h = t.wtile * kTileW + wave_w * 128 + b * 32 + 8 * q + 4 * kh;
      store4<Y>(y + static_cast<size_t>(prow) * a.H + h, v[q][0], v[q][1], v[q][2], v[q][3]);
    }
  }
}

// The fix-ups for ffn_tiled16_kernel's partial tiles (8x8 blocks of 16x16 per
// wave, block (i, j) at vectors (i * 8 + j) * 64 + lane). gate_up task (item,
// i < 4, j) sums gate block i and up block i + 4 of token block j over the
// parts (its tail is cut into up to 16 parts of few items: the parts' loads go
// out together); down task (item, i, jq) covers four token blocks 4 jq ..
// 4 jq + 3 (four independent loads per part in flight per lane; its tail has
// more items and fewer parts).
template <typename T>
__global__ __launch_bounds__(kThreads) void gate_up_tail_fixup16(const FfnArgs a) {
  const int n_t = a.tile_map[0];
  const int per_split = a.n_wtiles * n_t;
  const int nk = a.k_per_split / kSK;
  const WorkSplit ws = work_split(a.splits * per_split, a.grid, nk, a.part_units);
  const int tasks = ws.n_units / ws.S * 32;
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave;
  const int wave_w = wave >> 1, wave_t = wave & 1, lr = lane & 15, kq = lane >> 4;
  T* inter = static_cast<T*>(a.out);
  for (int task = blockIdx.x; task < tasks; task += gridDim.x) {
    const int it = task >> 5, i = (task >> 3) & 3, j = task & 7;
    const Tile t = decode_tile(a, ws.n_full + it, per_split, n_t, a.tile_rows);
    const f32x4* pp = reinterpret_cast<const f32x4*>(a.part) +
                      static_cast<size_t>(it * ws.S * 4 + wave) * kPartVecsPerWave + lane;
    f32x4 g = {}, u = {};
    // The parts of one block are independent loads: unrolled, up to 16 of
    // them are in flight per lane (the gate_up tail often splits 8 ways).
#pragma unroll 8
    for (int p = 0; p < ws.S; ++p) {
      g += pp[static_cast<size_t>(p) * 4 * kPartVecsPerWave + (i * 8 + j) * kWave];
      u += pp[static_cast<size_t>(p) * 4 * kPartVecsPerWave + ((i + 4) * 8 + j) * kWave];
    }
    const int col = t.wtile * (kTileW / 2) + wave_w * 64 + i * 16 + 4 * kq;
    const int prow = t.row0 + (2 * j + wave_t) * 16 + lr;
    if (prow < t.row_end)
      store4<T>(inter + static_cast<size_t>(prow) * a.I + col, gate_act_fast(a.act, g[0]) * u[0],
                gate_act_fast(a.act, g[1]) * u[1], gate_act_fast(a.act, g[2]) * u[2],
                gate_act_fast(a.act, g[3]) * u[3]);
  }
}

template <typename Y>
__global__ __launch_bounds__(kThreads) void down_tail_fixup16(const FfnArgs a) {
  const int n_t = a.tile_map[0];
  const int per_split = a.n_wtiles * n_t;
  const int nk = a.k_per_split / kSK;
  const WorkSplit ws = work_split(a.splits * per_split, a.grid, nk, a.part_units);
  const int tasks = ws.n_units / ws.S * 16;
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave;
  const int wave_w = wave >> 1, wave_t = wave & 1, lr = lane & 15, kq = lane >> 4;
  for (int task = blockIdx.x; task < tasks; task += gridDim.x) {
    const int it = task >> 4, i = (task >> 1) & 7, jq = task & 1;
    const Tile t = decode_tile(a, ws.n_full + it, per_split, n_t, a.tile_rows);
    f32x4 v[4] = {};
    for (int p = 0; p < ws.S; ++p) {
      const f32x4* pp = reinterpret_cast<const f32x4*>(a.part) +
                        static_cast<size_t>((it * ws.S + p) * 4 + wave) * kPartVecsPerWave + lane;
#pragma unroll
      for (int q = 0; q < 4; ++q) v[q] += pp[(i * 8 + 4 * jq + q) * kWave];
    }
    Y* y = static_cast<Y*>(a.out) + static_cast<size_t>(t.split) * a.R * a.H;
    const int h = t.wtile * kTileW + wave_w * 128 + i * 16 + 4 * kq;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int prow = t.row0 + (2 * (4 * jq + q) + wave_t) * 16 + lr;
      if (prow < t.row_end)
        store4<Y>(y + static_cast<size_t>(prow) * a.H + h, v[q][0], v[q][1], v[q][2], v[q][3]);
    }
  }
}

}  // namespace

// ffn_tiled16_kernel launches (the kRagged instance when a.ragged), one
// explicit instance per (dtype, projection) in its own object file
// (ffn_tiled16.hip): the kernel's K loop exists in one copy per token-block
// count, and the four instances compile in parallel.
template <typename T, bool kGateUp>
hipError_t launch_tiled16(const FfnArgs& a, hipStream_t s);

}  // namespace moe355
