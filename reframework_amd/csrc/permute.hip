// Stable counting sort of routed slots by expert.
//
// Replaces the grouping of fused_experts (reframework/moe/fused.py:70-80),
// which visits experts in ascending id and, inside an expert, slots in
// ascending flat (t,k) order. Two launches, no host round trip:
//   1. count:   each block histograms kPermuteChunk slots into LDS and writes
//               its per-expert counts (256 slots a block, one per thread: at
//               1024 a block ranked its slots in four dependent rounds, and
//               the scatter of 8192 slots ran on 8 CUs);
//   2. scatter: each block rebuilds the global expert starts and its own
//               prefix from the count table, ranks its slots stably with
//               wavefront ballots, and writes slot_to_row / row_src. Block 0
//               also writes expert_offsets and the tile map the expert-FFN
//               kernels are launched over.
// Only indices move here (4*T*K bytes each way); token rows are gathered later
// by the gate_up kernel straight from x, so no permuted copy of x is written.
#include "common.h"

namespace moe355 {
namespace {

constexpr int kThreads = 256;
constexpr int kRounds = kPermuteChunk / kThreads;            // count + scatter launches
constexpr int kSingleRounds = kPermuteSingleMax / kThreads;  // the one-block permute
constexpr int kWaves = kThreads / kWave;
static_assert(kMaxExperts <= 256, "the scatter ranks slots by the 8 bits of the expert id");

__global__ __launch_bounds__(kThreads) void count_kernel(const PermuteArgs a) {
  __shared__ int hist[kMaxExperts];
  const int b = blockIdx.x, tid = threadIdx.x;
  for (int e = tid; e < a.E; e += kThreads) hist[e] = 0;
  __syncthreads();
#pragma unroll
  for (int r = 0; r < kRounds; ++r) {
    const int slot = b * kPermuteChunk + r * kThreads + tid;
    if (slot < a.R) {
      const int e = routed_expert(a, slot);
      if (e >= 0) atomicAdd(&hist[e], 1);
    }
  }
  __syncthreads();
  for (int e = tid; e < a.E; e += kThreads) a.block_counts[b * a.E + e] = hist[e];
}

// kSingle: all slots fit one block (up to kPermuteSingleMax); the block counts
// them itself and the separate count launch is skipped.
template <bool kSingle>
__global__ __launch_bounds__(kThreads) void scatter_kernel(const PermuteArgs a) {
  __shared__ int base[kMaxExperts];     // first row of this block's slots of expert e
  __shared__ int start[kMaxExperts + 1];  // expert_offsets
  __shared__ int total[kMaxExperts];
  __shared__ int tile_start[kMaxExperts + 1];
  __shared__ int wave_cnt[kWaves][kMaxExperts];

  const int b = blockIdx.x, tid = threadIdx.x;
  const int lane = tid & (kWave - 1), wave = tid / kWave;

  if (kSingle) {
    for (int e = tid; e < a.E; e += kThreads) {
      total[e] = 0;
      base[e] = 0;
    }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < kSingleRounds; ++r) {
      const int slot = r * kThreads + tid;
      if (slot < a.R) {
        const int e = routed_expert(a, slot);
        if (e >= 0) atomicAdd(&total[e], 1);
      }
    }
  } else {
    // Slots of expert e in all blocks (total) and in the blocks before this
    // one (base), from the count table. Thread tid sums expert tid % E over
    // part tid / E of the blocks (P = min(256 / E, 8) parts; one part when
    // E > 128) with its loads unrolled, so they are in flight together; the
    // parts are added in LDS, at most 8 per expert. One thread per expert
    // walking every block paid one L2 round trip per block (32 for 64 experts
    // at 4096 tokens).
    __shared__ int ptot[kThreads], ppre[kThreads];
    const int P = min(kThreads / a.E, 8);
    const int e = tid % a.E, p = tid / a.E;
    int tot = 0, pre = 0;
    if (p < P) {
      const int per = (a.n_blocks + P - 1) / P;
      const int b1 = min(a.n_blocks, (p + 1) * per);
#pragma unroll 8
      for (int bb = p * per; bb < b1; ++bb) {
        const int c = a.block_counts[bb * a.E + e];
        tot += c;
        pre += bb < b ? c : 0;
      }
    }
    ptot[tid] = tot;
    ppre[tid] = pre;
    __syncthreads();
    for (int x = tid; x < a.E; x += kThreads) {
      int t2 = 0, p2 = 0;
      for (int q = 0; q < P; ++q) {
        t2 += ptot[q * a.E + x];
        p2 += ppre[q * a.E + x];
      }
      total[x] = t2;
      base[x] = p2;
    }
  }
  __syncthreads();
  if (wave == 0) {
    // Exclusive scans of the expert row counts and tile counts by one wave:
    // lane l owns experts l*per .. l*per+per-1 (per <= 4 for E <= 256).
    constexpr int kPer = kMaxExperts / kWave;
    const int per = (a.E + kWave - 1) / kWave;
    int cnt[kPer], tl[kPer];
    int sc = 0, st = 0;
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int e = lane * per + i;
      const bool own = i < per && e < a.E;
      cnt[i] = own ? total[e] : 0;
      tl[i] = (cnt[i] + a.tile_rows - 1) / a.tile_rows;
      sc += cnt[i];
      st += tl[i];
    }
    int ic = sc, it = st;  // inclusive scans across lanes
#pragma unroll
    for (int o = 1; o < kWave; o <<= 1) {
      const int vc = __shfl_up(ic, o, kWave), vt = __shfl_up(it, o, kWave);
      if (lane >= o) {
        ic += vc;
        it += vt;
      }
    }
    int ec = ic - sc, et = it - st;
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int e = lane * per + i;
      if (i < per && e < a.E) {
        start[e] = ec;
        tile_start[e] = et;
      }
      ec += cnt[i];
      et += tl[i];
    }
    if (lane == kWave - 1) {
      start[a.E] = ic;
      tile_start[a.E] = it < a.max_tiles ? it : a.max_tiles;
    }
  }
  __syncthreads();
  for (int e = tid; e < a.E; e += kThreads) base[e] += start[e];

  if (b == 0) {
    for (int e = tid; e <= a.E; e += kThreads) a.offsets[e] = start[e];
    // The tile map lists the experts' tiles in an interleaved order of their
    // sizes (largest, smallest, second largest, second smallest, ..; ties by
    // expert id), so the GEMMs' rounds mix weight-stream-bound items of small
    // experts with MFMA-bound items of large ones: fine-grained 4096 tokens
    // gate_up -2 %, Phi-3.5 2048 tokens -2 %, Mixtral 4096 tokens down -2 %
    // against expert-id order. Rank r of the size order goes to place 2 r in
    // the first half, 2 (E - 1 - r) + 1 in the second.
    __shared__ int order[kMaxExperts];         // expert at place p
    __shared__ int place_start[kMaxExperts + 1];  // first tile of place p
    for (int e = tid; e < a.E; e += kThreads) {
      const int n = total[e];
      int r = 0;
      for (int f = 0; f < a.E; ++f) r += (total[f] > n || (total[f] == n && f < e)) ? 1 : 0;
      order[2 * r < a.E ? 2 * r : 2 * (a.E - 1 - r) + 1] = e;
    }
    __syncthreads();
    if (wave == 0) {
      constexpr int kPer = kMaxExperts / kWave;
      const int per = (a.E + kWave - 1) / kWave;
      int tl[kPer], st = 0;
#pragma unroll
      for (int i = 0; i < kPer; ++i) {
        const int q = lane * per + i;
        tl[i] = i < per && q < a.E ? (total[order[q]] + a.tile_rows - 1) / a.tile_rows : 0;
        st += tl[i];
      }
      int it = st;
#pragma unroll
      for (int o = 1; o < kWave; o <<= 1) {
        const int v = __shfl_up(it, o, kWave);
        if (lane >= o) it += v;
      }
      int et = it - st;
#pragma unroll
      for (int i = 0; i < kPer; ++i) {
        const int q = lane * per + i;
        if (i < per && q < a.E) place_start[q] = et;
        et += tl[i];
      }
      if (lane == kWave - 1) place_start[a.E] = it;
    }
    __syncthreads();
    const int ntiles = tile_start[a.E];
    if (tid == 0) {
      a.tile_map[0] = ntiles;
      a.tile_map[1] = a.tile_rows;
    }
    for (int j = tid; j < ntiles; j += kThreads) {
      int lo = 0, hi = a.E - 1;  // last place with place_start[p] <= j
      while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (place_start[mid] <= j) lo = mid; else hi = mid - 1;
      }
      const int e = order[lo];
      a.tile_map[2 + 2 * j] = e;
      a.tile_map[3 + 2 * j] =
          start[e] + (j - place_start[lo]) * tile_height(start[e + 1] - start[e], a.tile_rows);
    }
  }

  const unsigned long long lt_mask = (1ull << lane) - 1ull;
  // Rounds past the last routed slot have nothing to rank.
  constexpr int rounds = kSingle ? kSingleRounds : kRounds;
  for (int r = 0; r < rounds && b * kPermuteChunk + r * kThreads < a.R; ++r) {
    for (int i = tid; i < kWaves * a.E; i += kThreads) wave_cnt[i / a.E][i % a.E] = 0;
    __syncthreads();
    const int slot = b * kPermuteChunk + r * kThreads + tid;
    const int e = slot < a.R ? routed_expert(a, slot) : -1;
    // Lanes of this wave routed to the same expert: the routed lanes that
    // agree with this lane on each of the 8 bits of the expert id (E <= 256),
    // one ballot per bit instead of one per distinct expert. The rank is the
    // count of such lanes below this one; the lowest of them writes the
    // wave's count.
    unsigned long long same = __ballot(e >= 0);
#pragma unroll
    for (int bit = 0; bit < 8; ++bit) {
      const bool set = (e >> bit) & 1;
      const unsigned long long m = __ballot(set);
      same &= set ? m : ~m;
    }
    const int rank = __popcll(same & lt_mask);
    if (e >= 0 && rank == 0) wave_cnt[wave][e] = __popcll(same);
    __syncthreads();
    if (slot < a.R) {
      if (e >= 0) {
        int row = base[e] + rank;
        for (int w = 0; w < wave; ++w) row += wave_cnt[w][e];
        a.slot_to_row[slot] = row;
        a.row_src[row] = slot / a.K;
      } else {
        a.slot_to_row[slot] = -1;
      }
    }
    __syncthreads();
    for (int ee = tid; ee < a.E; ee += kThreads) {
      int add = 0;
      for (int w = 0; w < kWaves; ++w) add += wave_cnt[w][ee];
      base[ee] += add;
    }
    __syncthreads();
  }
}

}  // namespace

hipError_t launch_permute(const PermuteArgs& a, hipStream_t s) {
  if (a.R == 0) return hipSuccess;
  if (a.n_blocks == 1) {
    scatter_kernel<true><<<dim3(1), dim3(kThreads), 0, s>>>(a);
    return hipGetLastError();
  }
  count_kernel<<<dim3(a.n_blocks), dim3(kThreads), 0, s>>>(a);
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return err;
  scatter_kernel<false><<<dim3(a.n_blocks), dim3(kThreads), 0, s>>>(a);
  return hipGetLastError();
}

}  // namespace moe355
