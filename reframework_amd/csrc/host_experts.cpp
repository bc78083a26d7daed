// Host-side expert FFN for the CPU/GPU split forward (libmoe355_host.so).
//
// The reference computes the experts that are not resident in device memory
// on the CPU while the GPU runs the resident ones, and sums both halves
// (reframework/moe/moe_layer.py:523-627, fused.py:140-197, there with int8
// GEMMs). Here the host half reads the staged 16-bit weights directly and
// computes with the GPU kernels' numerics: fp32 products and sums for
// gate|up, the activated intermediate rounded once to the weight type, fp32
// down projection, and the routing weight applied in fp32 to each slot's y
// before it is added to an fp32 output row.
//
// moe355_host_experts_int8 restates the reference's int8 host half itself:
// symmetric per-tensor int8 codes for the weights (quantized once by
// moe355_host_quantize_int8) and for each expert's block of token rows and of
// intermediate rows, integer dot products (exact), dequantized in fp32 by the
// product of the two scales. It reads half the bytes of the 16-bit path.
//
// Decode-sized inputs (a few tokens per expert) make this a weight stream:
// every weight row is read once from host memory and multiplied against all
// of an expert's token rows, which stay in L1/L2. Rows are split over the
// OpenMP threads in fixed blocks, so results do not depend on the thread
// count. For bf16 weights on a CPU with AVX512-BF16, vdpbf16ps multiplies bf16
// pairs (exact products) into fp32 sums; otherwise AVX-512F or AVX2 + FMA
// convert bf16/f16 to fp32 exactly before the FMAs (checked at run time).

#include <immintrin.h>
#include <omp.h>

#include <cmath>
#include <cstdint>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/moe355_host.h"

namespace {

thread_local std::string g_err;

int fail(int code, const std::string& msg) {
  g_err = msg;
  return code;
}

inline float bf16_to_f32(uint16_t b) {
  uint32_t u = static_cast<uint32_t>(b) << 16;
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}

// Round to nearest even, NaN kept quiet.
inline uint16_t f32_to_bf16(float f) {
  uint32_t u;
  std::memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x40);
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

inline float round_to_type(float v, int dtype) {
  if (dtype == MOE355_HOST_BF16) return bf16_to_f32(f32_to_bf16(v));
  if (dtype == MOE355_HOST_F16) return _cvtsh_ss(_cvtss_sh(v, _MM_FROUND_TO_NEAREST_INT));
  return v;
}

inline float load_w(const void* base, size_t i, int dtype) {
  if (dtype == MOE355_HOST_BF16) return bf16_to_f32(static_cast<const uint16_t*>(base)[i]);
  if (dtype == MOE355_HOST_F16) return _cvtsh_ss(static_cast<const uint16_t*>(base)[i]);
  return static_cast<const float*>(base)[i];
}

inline float act_mul(int act, float g, float u) {
  float a;
  if (act == 0) {
    a = g / (1.0f + std::exp(-g));
  } else if (act == 1) {
    a = 0.5f * g * (1.0f + std::erf(g * 0.70710678118654752f));
  } else {
    const float c = 0.79788456080286536f;  // sqrt(2/pi)
    a = 0.5f * g * (1.0f + std::tanh(c * (g + 0.044715f * g * g * g)));
  }
  return a * u;
}

// ---------------------------------------------------------------- dot rows
// out[t * ldo + r] = sum_k a[t * n + k] * W[r * n + k] for r in [r0, r1),
// t in [0, m). a is fp32 (m rows of n), W rows are 16-bit or fp32.

constexpr int kMaxTok = 8;  // token rows per pass over a weight row
// Rows of W split in blocks of kRowBlock over the threads (static schedule).
constexpr int kRowBlock = 16;

template <int DT>
__attribute__((target("avx512f,avx512bw")))
inline __m512 load16_avx512(const void* w, size_t i) {
  if constexpr (DT == MOE355_HOST_BF16) {
    __m256i h = _mm256_loadu_si256(reinterpret_cast<const __m256i*>(
        static_cast<const uint16_t*>(w) + i));
    return _mm512_castsi512_ps(_mm512_slli_epi32(_mm512_cvtepu16_epi32(h), 16));
  } else if constexpr (DT == MOE355_HOST_F16) {
    __m256i h = _mm256_loadu_si256(reinterpret_cast<const __m256i*>(
        static_cast<const uint16_t*>(w) + i));
    return _mm512_cvtph_ps(h);
  } else {
    return _mm512_loadu_ps(static_cast<const float*>(w) + i);
  }
}

// Ask for the row's next K block (its cache lines) while this one is
// multiplied: with the K blocking each weight row is read in short runs, which
// the hardware prefetchers follow poorly.
template <int DT>
inline void prefetch_next_block(const void* w, size_t row, int k0, int n) {
  constexpr int esz = DT == MOE355_HOST_F32 ? 4 : 2;
  const char* p = static_cast<const char*>(w) + (row + k0) * esz;
  const int bytes = ((n - k0) < 512 ? (n - k0) : 512) * esz;
  for (int off = 0; off < bytes; off += 64) _mm_prefetch(p + off, _MM_HINT_T0);
}

// K is walked in blocks of kKBlock so that the MT token rows' block (MT x
// kKBlock fp32, 16 KB at 8 tokens) stays in L1 while the 16 weight rows of a
// row block stream past it; each (row, token) partial is reduced per block.
constexpr int kKBlock = 512;

template <int MT, int DT>
__attribute__((target("avx512f,avx512bw")))
void dot_block_avx512(const float* a, int lda, int n, const void* w, int r0, int r1,
                      float* out, int ldo) {
  float part[16][MT];
  for (int r = 0; r < r1 - r0; ++r)
    for (int t = 0; t < MT; ++t) part[r][t] = 0.0f;
  for (int kb = 0; kb < n; kb += kKBlock) {
    const int ke = (kb + kKBlock) < n ? (kb + kKBlock) : n;
    const int kv = kb + ((ke - kb) & ~15);
    for (int r = r0; r < r1; ++r) {
      const size_t row = static_cast<size_t>(r) * n;
      prefetch_next_block<DT>(w, row, ke, n);
      __m512 acc[MT];
      for (int t = 0; t < MT; ++t) acc[t] = _mm512_setzero_ps();
      for (int k = kb; k < kv; k += 16) {
        const __m512 wv = load16_avx512<DT>(w, row + k);
        for (int t = 0; t < MT; ++t)
          acc[t] = _mm512_fmadd_ps(wv, _mm512_loadu_ps(a + (size_t)t * lda + k), acc[t]);
      }
      for (int t = 0; t < MT; ++t) {
        float s = _mm512_reduce_add_ps(acc[t]);
        for (int k = kv; k < ke; ++k) s += load_w(w, row + k, DT) * a[(size_t)t * lda + k];
        part[r - r0][t] += s;
      }
    }
  }
  for (int r = r0; r < r1; ++r)
    for (int t = 0; t < MT; ++t) out[(size_t)t * ldo + r] = part[r - r0][t];
}

template <int MT>
__attribute__((target("avx512f,avx512bw")))
void dot_block_dt_avx512(const float* a, int lda, int n, const void* w, int dtype, int r0,
                      int r1, float* out, int ldo) {
  if (dtype == MOE355_HOST_BF16)
    dot_block_avx512<MT, MOE355_HOST_BF16>(a, lda, n, w, r0, r1, out, ldo);
  else if (dtype == MOE355_HOST_F16)
    dot_block_avx512<MT, MOE355_HOST_F16>(a, lda, n, w, r0, r1, out, ldo);
  else
    dot_block_avx512<MT, MOE355_HOST_F32>(a, lda, n, w, r0, r1, out, ldo);
}

__attribute__((target("avx512f,avx512bw")))
void dot_rows_avx512(const float* a, int lda, int m, int n, const void* w, int dtype, int r0, int r1,
                     float* out, int ldo) {
  for (int t0 = 0; t0 < m; t0 += kMaxTok) {
    const float* at = a + (size_t)t0 * lda;
    float* ot = out + (size_t)t0 * ldo;
    switch ((m - t0) < kMaxTok ? (m - t0) : kMaxTok) {
      case 1: dot_block_dt_avx512<1>(at, lda, n, w, dtype, r0, r1, ot, ldo); break;
      case 2: dot_block_dt_avx512<2>(at, lda, n, w, dtype, r0, r1, ot, ldo); break;
      case 3: dot_block_dt_avx512<3>(at, lda, n, w, dtype, r0, r1, ot, ldo); break;
      case 4: dot_block_dt_avx512<4>(at, lda, n, w, dtype, r0, r1, ot, ldo); break;
      case 5: dot_block_dt_avx512<5>(at, lda, n, w, dtype, r0, r1, ot, ldo); break;
      case 6: dot_block_dt_avx512<6>(at, lda, n, w, dtype, r0, r1, ot, ldo); break;
      case 7: dot_block_dt_avx512<7>(at, lda, n, w, dtype, r0, r1, ot, ldo); break;
      default: dot_block_dt_avx512<8>(at, lda, n, w, dtype, r0, r1, ot, ldo); break;
    }
  }
}

// bf16 weights against bf16 token rows with vdpbf16ps: each instruction
// multiplies 32 bf16 pairs (products exact in fp32) and adds them to 16 fp32
// sums, half the instructions of convert + FMA per weight. The intermediate
// is already rounded to bf16, so the token rows lose nothing. R weight rows
// at a time, so one token vector feeds R instructions (R = 2 at 5-8 tokens,
// 4 below); each (row, token) keeps its 16 lane sums across K blocks in vpart
// and they are added across lanes once per row.
template <int MT, int R>
__attribute__((target("avx512f,avx512bw,avx512bf16")))
inline void dot_rows_r_bf16dp(const uint16_t* a, int lda, int kb, int ke, int kv, const uint16_t* w,
                              int n, int r, __m512 (*vpart)[MT], float (*part)[MT]) {
  const uint16_t* wr[R];
#pragma GCC unroll 4
  for (int q = 0; q < R; ++q) {
    wr[q] = w + static_cast<size_t>(r + q) * n;
    prefetch_next_block<MOE355_HOST_BF16>(w, static_cast<size_t>(r + q) * n, ke, n);
  }
  __m512 acc[R][MT];
#pragma GCC unroll 4
  for (int q = 0; q < R; ++q)
#pragma GCC unroll 8
    for (int t = 0; t < MT; ++t) acc[q][t] = vpart[q][t];
  for (int k = kb; k < kv; k += 32) {
    __m512bh wv[R];
#pragma GCC unroll 4
    for (int q = 0; q < R; ++q) wv[q] = (__m512bh)_mm512_loadu_si512(wr[q] + k);
#pragma GCC unroll 8
    for (int t = 0; t < MT; ++t) {
      const __m512bh av = (__m512bh)_mm512_loadu_si512(a + (size_t)t * lda + k);
#pragma GCC unroll 4
      for (int q = 0; q < R; ++q) acc[q][t] = _mm512_dpbf16_ps(acc[q][t], wv[q], av);
    }
  }
#pragma GCC unroll 4
  for (int q = 0; q < R; ++q)
#pragma GCC unroll 8
    for (int t = 0; t < MT; ++t) {
      vpart[q][t] = acc[q][t];
      for (int k = kv; k < ke; ++k)
        part[q][t] += bf16_to_f32(wr[q][k]) * bf16_to_f32(a[(size_t)t * lda + k]);
    }
}

template <int MT>
__attribute__((target("avx512f,avx512bw,avx512bf16")))
void dot_block_bf16dp(const uint16_t* a, int lda, int n, const uint16_t* w, int r0, int r1,
                      float* out, int ldo) {
  constexpr int R = MT > 4 ? 2 : 4;
  __m512 vpart[kRowBlock][MT];
  float part[kRowBlock][MT];
  for (int r = 0; r < r1 - r0; ++r)
    for (int t = 0; t < MT; ++t) {
      vpart[r][t] = _mm512_setzero_ps();
      part[r][t] = 0.0f;
    }
  for (int kb = 0; kb < n; kb += kKBlock) {
    const int ke = (kb + kKBlock) < n ? (kb + kKBlock) : n;
    const int kv = kb + ((ke - kb) & ~31);
    int r = r0;
    for (; r + R <= r1; r += R)
      dot_rows_r_bf16dp<MT, R>(a, lda, kb, ke, kv, w, n, r, &vpart[r - r0], &part[r - r0]);
    for (; r < r1; ++r)
      dot_rows_r_bf16dp<MT, 1>(a, lda, kb, ke, kv, w, n, r, &vpart[r - r0], &part[r - r0]);
  }
  for (int r = r0; r < r1; ++r)
    for (int t = 0; t < MT; ++t)
      out[(size_t)t * ldo + r] = _mm512_reduce_add_ps(vpart[r - r0][t]) + part[r - r0][t];
}

__attribute__((target("avx512f,avx512bw,avx512bf16")))
void dot_rows_bf16dp(const uint16_t* a, int lda, int m, int n, const uint16_t* w, int r0, int r1,
                     float* out, int ldo) {
  for (int t0 = 0; t0 < m; t0 += kMaxTok) {
    const uint16_t* at = a + (size_t)t0 * lda;
    float* ot = out + (size_t)t0 * ldo;
    switch ((m - t0) < kMaxTok ? (m - t0) : kMaxTok) {
      case 1: dot_block_bf16dp<1>(at, lda, n, w, r0, r1, ot, ldo); break;
      case 2: dot_block_bf16dp<2>(at, lda, n, w, r0, r1, ot, ldo); break;
      case 3: dot_block_bf16dp<3>(at, lda, n, w, r0, r1, ot, ldo); break;
      case 4: dot_block_bf16dp<4>(at, lda, n, w, r0, r1, ot, ldo); break;
      case 5: dot_block_bf16dp<5>(at, lda, n, w, r0, r1, ot, ldo); break;
      case 6: dot_block_bf16dp<6>(at, lda, n, w, r0, r1, ot, ldo); break;
      case 7: dot_block_bf16dp<7>(at, lda, n, w, r0, r1, ot, ldo); break;
      default: dot_block_bf16dp<8>(at, lda, n, w, r0, r1, ot, ldo); break;
    }
  }
}

template <int DT>
__attribute__((target("avx2,fma,f16c")))
inline __m256 load8_avx2(const void* w, size_t i) {
  if constexpr (DT == MOE355_HOST_BF16) {
    __m128i h = _mm_loadu_si128(reinterpret_cast<const __m128i*>(
        static_cast<const uint16_t*>(w) + i));
    return _mm256_castsi256_ps(_mm256_slli_epi32(_mm256_cvtepu16_epi32(h), 16));
  } else if constexpr (DT == MOE355_HOST_F16) {
    __m128i h = _mm_loadu_si128(reinterpret_cast<const __m128i*>(
        static_cast<const uint16_t*>(w) + i));
    return _mm256_cvtph_ps(h);
  } else {
    return _mm256_loadu_ps(static_cast<const float*>(w) + i);
  }
}

__attribute__((target("avx2,fma,f16c")))
inline float hsum_avx2(__m256 v) {
  __m128 s = _mm_add_ps(_mm256_castps256_ps128(v), _mm256_extractf128_ps(v, 1));
  s = _mm_add_ps(s, _mm_movehl_ps(s, s));
  s = _mm_add_ss(s, _mm_movehdup_ps(s));
  return _mm_cvtss_f32(s);
}

template <int MT, int DT>
__attribute__((target("avx2,fma,f16c")))
void dot_block_avx2(const float* a, int lda, int n, const void* w, int r0, int r1,
                    float* out, int ldo) {
  float part[16][MT];
  for (int r = 0; r < r1 - r0; ++r)
    for (int t = 0; t < MT; ++t) part[r][t] = 0.0f;
  for (int kb = 0; kb < n; kb += kKBlock) {
    const int ke = (kb + kKBlock) < n ? (kb + kKBlock) : n;
    const int kv = kb + ((ke - kb) & ~7);
    for (int r = r0; r < r1; ++r) {
      const size_t row = static_cast<size_t>(r) * n;
      prefetch_next_block<DT>(w, row, ke, n);
      __m256 acc[MT];
      for (int t = 0; t < MT; ++t) acc[t] = _mm256_setzero_ps();
      for (int k = kb; k < kv; k += 8) {
        const __m256 wv = load8_avx2<DT>(w, row + k);
        for (int t = 0; t < MT; ++t)
          acc[t] = _mm256_fmadd_ps(wv, _mm256_loadu_ps(a + (size_t)t * lda + k), acc[t]);
      }
      for (int t = 0; t < MT; ++t) {
        float s = hsum_avx2(acc[t]);
        for (int k = kv; k < ke; ++k) s += load_w(w, row + k, DT) * a[(size_t)t * lda + k];
        part[r - r0][t] += s;
      }
    }
  }
  for (int r = r0; r < r1; ++r)
    for (int t = 0; t < MT; ++t) out[(size_t)t * ldo + r] = part[r - r0][t];
}

template <int MT>
__attribute__((target("avx2,fma,f16c")))
void dot_block_dt_avx2(const float* a, int lda, int n, const void* w, int dtype, int r0,
                      int r1, float* out, int ldo) {
  if (dtype == MOE355_HOST_BF16)
    dot_block_avx2<MT, MOE355_HOST_BF16>(a, lda, n, w, r0, r1, out, ldo);
  else if (dtype == MOE355_HOST_F16)
    dot_block_avx2<MT, MOE355_HOST_F16>(a, lda, n, w, r0, r1, out, ldo);
  else
    dot_block_avx2<MT, MOE355_HOST_F32>(a, lda, n, w, r0, r1, out, ldo);
}

__attribute__((target("avx2,fma,f16c")))
void dot_rows_avx2(const float* a, int lda, int m, int n, const void* w, int dtype, int r0, int r1,
                   float* out, int ldo) {
  constexpr int kTok = 4;
  for (int t0 = 0; t0 < m; t0 += kTok) {
    const float* at = a + (size_t)t0 * lda;
    float* ot = out + (size_t)t0 * ldo;
    switch ((m - t0) < kTok ? (m - t0) : kTok) {
      case 1: dot_block_dt_avx2<1>(at, lda, n, w, dtype, r0, r1, ot, ldo); break;
      case 2: dot_block_dt_avx2<2>(at, lda, n, w, dtype, r0, r1, ot, ldo); break;
      case 3: dot_block_dt_avx2<3>(at, lda, n, w, dtype, r0, r1, ot, ldo); break;
      default: dot_block_dt_avx2<4>(at, lda, n, w, dtype, r0, r1, ot, ldo); break;
    }
  }
}

bool have_avx512() {
  static const bool ok = __builtin_cpu_supports("avx512f") && __builtin_cpu_supports("avx512bw");
  return ok;
}

bool have_avx512bf16() {
  static const bool ok = have_avx512() && __builtin_cpu_supports("avx512bf16");
  return ok;
}

bool have_avx2() {
  static const bool ok = __builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma") &&
                         __builtin_cpu_supports("f16c");
  return ok;
}

// Instruction set used: the best the CPU has, capped by MOE355_HOST_ISA
// (avx2 | avx512 | avx512bf16; read per call, so one process can compare the
// paths).
enum Isa { kAvx2 = 0, kAvx512 = 1, kAvx512Bf16 = 2 };

Isa isa() {
  Isa best = have_avx512bf16() ? kAvx512Bf16 : (have_avx512() ? kAvx512 : kAvx2);
  const char* e = std::getenv("MOE355_HOST_ISA");
  if (e && std::strcmp(e, "avx2") == 0) return kAvx2;
  if (e && std::strcmp(e, "avx512") == 0 && best > kAvx512) return kAvx512;
  return best;
}

// a: the token rows in fp32 (lda floats apart); a16: the same rows as bf16
// bits (lda16 elements apart), used by the vdpbf16ps path for bf16 weights.
void dot_rows(const float* a, int lda, const uint16_t* a16, int lda16, int m, int n,
              const void* w, int dtype, int rows, float* out, int ldo, int n_threads, Isa use) {
  const int blocks = (rows + kRowBlock - 1) / kRowBlock;
  const bool dp = use == kAvx512Bf16 && dtype == MOE355_HOST_BF16;
#pragma omp parallel for schedule(static) num_threads(n_threads)
  for (int b = 0; b < blocks; ++b) {
    const int r0 = b * kRowBlock;
    const int r1 = (r0 + kRowBlock) < rows ? (r0 + kRowBlock) : rows;
    if (dp)
      dot_rows_bf16dp(a16, lda16, m, n, static_cast<const uint16_t*>(w), r0, r1, out, ldo);
    else if (use >= kAvx512)
      dot_rows_avx512(a, lda, m, n, w, dtype, r0, r1, out, ldo);
    else
      dot_rows_avx2(a, lda, m, n, w, dtype, r0, r1, out, ldo);
  }
}

// ------------------------------------------------------------------- int8
// Symmetric per-tensor codes of n fp32 values (the reference's
// _sym_int8_quantize, reframework/moe/offload_cache.py:58-72): amax = max |v|;
// amax <= 0 gives zero codes and scale 1; otherwise scale = amax / 127 in fp32
// and code = clamp(round_half_even(v / scale), -127, 127), the division in
// fp32 (torch's true division). Returns the scale.
template <typename Get>
float quantize_codes(size_t n, Get get, int8_t* q, int n_threads) {
  float amax = 0.0f;
#pragma omp parallel for reduction(max : amax) schedule(static) num_threads(n_threads) if (n > (1u << 14))
  for (size_t i = 0; i < n; ++i) {
    const float a = std::fabs(get(i));
    if (a > amax) amax = a;
  }
  if (!(amax > 0.0f)) {
    std::memset(q, 0, n);
    return 1.0f;
  }
  const float scale = amax / 127.0f;
#pragma omp parallel for schedule(static) num_threads(n_threads) if (n > (1u << 14))
  for (size_t i = 0; i < n; ++i) {
    float c = std::nearbyint(get(i) / scale);
    c = c < -127.0f ? -127.0f : (c > 127.0f ? 127.0f : c);
    q[i] = static_cast<int8_t>(c);
  }
  return scale;
}

// Dequantization multiplier of an int32 dot product: torch multiplies the
// fp32 tensor by the Python float xs * s (a double product), which it casts
// to fp32 first.
inline float dequant_mul(float xs, float s) {
  return static_cast<float>(static_cast<double>(xs) * static_cast<double>(s));
}

// Longest K of an int8 product: (code + 128) * w sums stay below 2^31.
constexpr int kMaxInt8K = 65536;

// Token rows of an int8 product are stored as unsigned codes (code + 128),
// lda bytes apart: vpdpbusd multiplies unsigned by signed bytes, and the
// excess 128 * sum_k w[r, k] is taken off with the weight row's code sum.
constexpr int kKBlock8 = 1024;

// R weight rows at a time against MT token rows: each token vector loaded
// from L1 feeds R vpdpbusd, so the loads per product drop from (MT + 1) / MT
// to (MT + R) / (R * MT) (R * MT accumulators; R = 2 at 5-8 tokens, 4 below).
// The 16 lane sums of each (row, token) are carried across K blocks in vpart
// and reduced across lanes once per row (integer sums: any order is exact);
// a reduction per K block cost about as many instructions as the products of
// the block at 8 tokens.
template <int MT, int R>
__attribute__((target("avx512f,avx512bw,avx512vnni")))
inline void dot8_rows_r_vnni(const uint8_t* a, int lda, int kb, int ke, int kv, const int8_t* w,
                             int n, int r, __m512i (*vpart)[MT], int32_t (*part)[MT]) {
  const int8_t* wr[R];
  for (int q = 0; q < R; ++q) {
    wr[q] = w + static_cast<size_t>(r + q) * n;
    for (int off = ke; off < ((ke + kKBlock8) < n ? (ke + kKBlock8) : n); off += 64)
      _mm_prefetch(reinterpret_cast<const char*>(wr[q] + off), _MM_HINT_T0);
  }
  __m512i acc[R][MT];
#pragma GCC unroll 4
  for (int q = 0; q < R; ++q)
#pragma GCC unroll 8
    for (int t = 0; t < MT; ++t) acc[q][t] = vpart[q][t];
  for (int k = kb; k < kv; k += 64) {
    __m512i wv[R];
#pragma GCC unroll 4
    for (int q = 0; q < R; ++q) wv[q] = _mm512_loadu_si512(wr[q] + k);
#pragma GCC unroll 8
    for (int t = 0; t < MT; ++t) {
      const __m512i av = _mm512_loadu_si512(a + (size_t)t * lda + k);
#pragma GCC unroll 4
      for (int q = 0; q < R; ++q) acc[q][t] = _mm512_dpbusd_epi32(acc[q][t], av, wv[q]);
    }
  }
#pragma GCC unroll 4
  for (int q = 0; q < R; ++q)
#pragma GCC unroll 8
    for (int t = 0; t < MT; ++t) {
      vpart[q][t] = acc[q][t];
      int32_t s = 0;
      for (int k = kv; k < ke; ++k) s += static_cast<int32_t>(a[(size_t)t * lda + k]) * wr[q][k];
      part[q][t] += s;
    }
}

template <int MT>
__attribute__((target("avx512f,avx512bw,avx512vnni")))
void dot8_block_vnni(const uint8_t* a, int lda, int n, const int8_t* w, const int32_t* rsum,
                     int r0, int r1, int32_t* out, int ldo) {
  constexpr int R = MT > 4 ? 2 : 4;
  __m512i vpart[kRowBlock][MT];
  int32_t part[kRowBlock][MT];
  for (int r = 0; r < r1 - r0; ++r)
    for (int t = 0; t < MT; ++t) {
      vpart[r][t] = _mm512_setzero_si512();
      part[r][t] = 0;
    }
  for (int kb = 0; kb < n; kb += kKBlock8) {
    const int ke = (kb + kKBlock8) < n ? (kb + kKBlock8) : n;
    const int kv = kb + ((ke - kb) & ~63);
    int r = r0;
    for (; r + R <= r1; r += R)
      dot8_rows_r_vnni<MT, R>(a, lda, kb, ke, kv, w, n, r, &vpart[r - r0], &part[r - r0]);
    for (; r < r1; ++r)
      dot8_rows_r_vnni<MT, 1>(a, lda, kb, ke, kv, w, n, r, &vpart[r - r0], &part[r - r0]);
  }
  for (int r = r0; r < r1; ++r)
    for (int t = 0; t < MT; ++t)
      out[(size_t)t * ldo + r] =
          _mm512_reduce_add_epi32(vpart[r - r0][t]) + part[r - r0][t] - 128 * rsum[r];
}

__attribute__((target("avx512f,avx512bw,avx512vnni")))
void dot8_rows_vnni(const uint8_t* a, int lda, int m, int n, const int8_t* w, const int32_t* rsum,
                    int r0, int r1, int32_t* out, int ldo) {
  for (int t0 = 0; t0 < m; t0 += kMaxTok) {
    const uint8_t* at = a + (size_t)t0 * lda;
    int32_t* ot = out + (size_t)t0 * ldo;
    switch ((m - t0) < kMaxTok ? (m - t0) : kMaxTok) {
      case 1: dot8_block_vnni<1>(at, lda, n, w, rsum, r0, r1, ot, ldo); break;
      case 2: dot8_block_vnni<2>(at, lda, n, w, rsum, r0, r1, ot, ldo); break;
      case 3: dot8_block_vnni<3>(at, lda, n, w, rsum, r0, r1, ot, ldo); break;
      case 4: dot8_block_vnni<4>(at, lda, n, w, rsum, r0, r1, ot, ldo); break;
      case 5: dot8_block_vnni<5>(at, lda, n, w, rsum, r0, r1, ot, ldo); break;
      case 6: dot8_block_vnni<6>(at, lda, n, w, rsum, r0, r1, ot, ldo); break;
      case 7: dot8_block_vnni<7>(at, lda, n, w, rsum, r0, r1, ot, ldo); break;
      default: dot8_block_vnni<8>(at, lda, n, w, rsum, r0, r1, ot, ldo); break;
    }
  }
}

// Without VNNI: both codes widened to int16 and multiplied by vpmaddwd (exact
// int32 pair sums), so no code-sum correction is needed.
template <int MT>
__attribute__((target("avx2,fma,f16c")))
void dot8_block_avx2(const uint8_t* a, int lda, int n, const int8_t* w, int r0, int r1,
                     int32_t* out, int ldo) {
  const __m256i bias = _mm256_set1_epi16(128);
  int32_t part[16][MT];
  for (int r = 0; r < r1 - r0; ++r)
    for (int t = 0; t < MT; ++t) part[r][t] = 0;
  for (int kb = 0; kb < n; kb += kKBlock8) {
    const int ke = (kb + kKBlock8) < n ? (kb + kKBlock8) : n;
    const int kv = kb + ((ke - kb) & ~15);
    for (int r = r0; r < r1; ++r) {
      const int8_t* wr = w + static_cast<size_t>(r) * n;
      for (int off = ke; off < ((ke + kKBlock8) < n ? (ke + kKBlock8) : n); off += 64)
        _mm_prefetch(reinterpret_cast<const char*>(wr + off), _MM_HINT_T0);
      __m256i acc[MT];
      for (int t = 0; t < MT; ++t) acc[t] = _mm256_setzero_si256();
      for (int k = kb; k < kv; k += 16) {
        const __m256i wv =
            _mm256_cvtepi8_epi16(_mm_loadu_si128(reinterpret_cast<const __m128i*>(wr + k)));
        for (int t = 0; t < MT; ++t) {
          const __m256i av = _mm256_sub_epi16(
              _mm256_cvtepu8_epi16(
                  _mm_loadu_si128(reinterpret_cast<const __m128i*>(a + (size_t)t * lda + k))),
              bias);
          acc[t] = _mm256_add_epi32(acc[t], _mm256_madd_epi16(av, wv));
        }
      }
      for (int t = 0; t < MT; ++t) {
        __m128i s4 = _mm_add_epi32(_mm256_castsi256_si128(acc[t]), _mm256_extracti128_si256(acc[t], 1));
        s4 = _mm_add_epi32(s4, _mm_shuffle_epi32(s4, 0x4e));
        s4 = _mm_add_epi32(s4, _mm_shuffle_epi32(s4, 0xb1));
        int32_t s = _mm_cvtsi128_si32(s4);
        for (int k = kv; k < ke; ++k)
          s += (static_cast<int32_t>(a[(size_t)t * lda + k]) - 128) * wr[k];
        part[r - r0][t] += s;
      }
    }
  }
  for (int r = r0; r < r1; ++r)
    for (int t = 0; t < MT; ++t) out[(size_t)t * ldo + r] = part[r - r0][t];
}

__attribute__((target("avx2,fma,f16c")))
void dot8_rows_avx2(const uint8_t* a, int lda, int m, int n, const int8_t* w, int r0, int r1,
                    int32_t* out, int ldo) {
  constexpr int kTok = 4;
  for (int t0 = 0; t0 < m; t0 += kTok) {
    const uint8_t* at = a + (size_t)t0 * lda;
    int32_t* ot = out + (size_t)t0 * ldo;
    switch ((m - t0) < kTok ? (m - t0) : kTok) {
      case 1: dot8_block_avx2<1>(at, lda, n, w, r0, r1, ot, ldo); break;
      case 2: dot8_block_avx2<2>(at, lda, n, w, r0, r1, ot, ldo); break;
      case 3: dot8_block_avx2<3>(at, lda, n, w, r0, r1, ot, ldo); break;
      default: dot8_block_avx2<4>(at, lda, n, w, r0, r1, ot, ldo); break;
    }
  }
}

bool have_avx512vnni() {
  static const bool ok = have_avx512() && __builtin_cpu_supports("avx512vnni");
  return ok;
}

// out[t * ldo + r] = sum_k (a[t, k] - 128) * w[r, k], exact in int32 (|sum|
// <= n * 127 * 127).
void dot8_rows(const uint8_t* a, int lda, int m, int n, const int8_t* w, const int32_t* rsum,
               int rows, int32_t* out, int ldo, int n_threads, Isa use) {
  const int blocks = (rows + kRowBlock - 1) / kRowBlock;
  const bool vnni = use >= kAvx512 && have_avx512vnni();
#pragma omp parallel for schedule(static) num_threads(n_threads)
  for (int b = 0; b < blocks; ++b) {
    const int r0 = b * kRowBlock;
    const int r1 = (r0 + kRowBlock) < rows ? (r0 + kRowBlock) : rows;
    if (vnni)
      dot8_rows_vnni(a, lda, m, n, w, rsum, r0, r1, out, ldo);
    else
      dot8_rows_avx2(a, lda, m, n, w, r0, r1, out, ldo);
  }
}

// Codes of m fp32 rows of n (contiguous) as unsigned bytes, lda apart.
float quantize_rows_u8(const float* v, int m, int n, uint8_t* out, int lda,
                       std::vector<int8_t>& tmp, int n_threads) {
  const size_t total = static_cast<size_t>(m) * n;
  tmp.resize(total);
  const float s = quantize_codes(total, [&](size_t i) { return v[i]; }, tmp.data(), n_threads);
#pragma omp parallel for schedule(static) num_threads(n_threads) if (total > (1u << 14))
  for (size_t i = 0; i < total; ++i)
    out[(i / n) * lda + i % n] = static_cast<uint8_t>(tmp[i] + 128);
  return s;
}

// row_sums[r] = sum of row r's int8 codes (exact in int32 for cols < 2^24)
void code_row_sums(const int8_t* q, int rows, int cols, int32_t* row_sums, int n_threads) {
#pragma omp parallel for schedule(static) num_threads(n_threads)
  for (int r = 0; r < rows; ++r) {
    int32_t sum = 0;
    const int8_t* qr = q + static_cast<size_t>(r) * cols;
    for (int c = 0; c < cols; ++c) sum += qr[c];
    row_sums[r] = sum;
  }
}

}  // namespace

extern "C" {

int moe355_host_quantize_int8(const void* w, int rows, int cols, int dtype, int8_t* q,
                              float* scale, int32_t* row_sums, int n_threads) {
  if (!w || !q || !scale || !row_sums) return fail(MOE355_HOST_EINVAL, "null pointer argument");
  if (rows <= 0 || cols <= 0) return fail(MOE355_HOST_EINVAL, "bad sizes");
  if (dtype != MOE355_HOST_F32 && dtype != MOE355_HOST_BF16 && dtype != MOE355_HOST_F16)
    return fail(MOE355_HOST_EINVAL, "dtype must be f32, bf16 or f16");
  if (n_threads <= 0) n_threads = omp_get_max_threads();
  const size_t n = static_cast<size_t>(rows) * cols;
  *scale = quantize_codes(n, [&](size_t i) { return load_w(w, i, dtype); }, q, n_threads);
  code_row_sums(q, rows, cols, row_sums, n_threads);
  return 0;
}

int moe355_host_int8_row_sums(const int8_t* q, int rows, int cols, int32_t* row_sums,
                              int n_threads) {
  if (!q || !row_sums) return fail(MOE355_HOST_EINVAL, "null pointer argument");
  if (rows <= 0 || cols <= 0) return fail(MOE355_HOST_EINVAL, "bad sizes");
  if (n_threads <= 0) n_threads = omp_get_max_threads();
  code_row_sums(q, rows, cols, row_sums, n_threads);
  return 0;
}

int moe355_host_experts_int8(const void* x, int T, int H, int I, int dtype, int n_experts,
                             const int8_t* const* w1q, const int8_t* const* w2q, const float* s1,
                             const float* s2, const int32_t* const* rs1,
                             const int32_t* const* rs2, const int32_t* slot_offsets,
                             const int32_t* slot_tokens, const float* slot_weights, int act,
                             int n_threads, float* out) {
  if (!x || !out || !slot_offsets ||
      (n_experts > 0 && (!w1q || !w2q || !s1 || !s2 || !rs1 || !rs2 || !slot_tokens ||
                         !slot_weights)))
    return fail(MOE355_HOST_EINVAL, "null pointer argument");
  if (T < 0 || H <= 0 || I <= 0 || n_experts < 0)
    return fail(MOE355_HOST_EINVAL, "bad sizes");
  // the biased products (code + 128) * w sum to at most n * 255 * 127 in int32
  if (H > kMaxInt8K || I > kMaxInt8K)
    return fail(MOE355_HOST_EINVAL, "H and I must be at most 65536 for the int8 products");
  if (dtype != MOE355_HOST_F32 && dtype != MOE355_HOST_BF16 && dtype != MOE355_HOST_F16)
    return fail(MOE355_HOST_EINVAL, "dtype must be f32, bf16 or f16");
  if (act < 0 || act > 2) return fail(MOE355_HOST_EINVAL, "unknown activation code");
  if (!have_avx2()) return fail(MOE355_HOST_ECPU, "the host CPU lacks AVX2/FMA/F16C");
  if (slot_offsets[0] != 0) return fail(MOE355_HOST_EINVAL, "slot_offsets[0] must be 0");
  for (int e = 0; e < n_experts; ++e) {
    if (slot_offsets[e + 1] < slot_offsets[e])
      return fail(MOE355_HOST_EINVAL, "slot_offsets must be non-decreasing");
    if (!w1q[e] || !w2q[e] || !rs1[e] || !rs2[e])
      return fail(MOE355_HOST_EINVAL, "null expert weight pointer");
  }
  const int n_slots = n_experts > 0 ? slot_offsets[n_experts] : 0;
  for (int s = 0; s < n_slots; ++s)
    if (slot_tokens[s] < 0 || slot_tokens[s] >= T)
      return fail(MOE355_HOST_EINVAL, "slot token index out of range");
  if (n_threads <= 0) n_threads = omp_get_max_threads();
  const Isa use = isa();

  std::vector<float> xa, inter, row;
  std::vector<int32_t> acc1, acc2;
  std::vector<uint8_t> xq, iq;
  std::vector<int8_t> tmp;
  for (int e = 0; e < n_experts; ++e) {
    const int s0 = slot_offsets[e], m = slot_offsets[e + 1] - s0;
    if (m == 0) continue;
    // the expert's token rows in fp32, then their codes (one scale for the block)
    xa.resize(static_cast<size_t>(m) * H);
    for (int j = 0; j < m; ++j) {
      const size_t src = static_cast<size_t>(slot_tokens[s0 + j]) * H;
      for (int h = 0; h < H; ++h) xa[(size_t)j * H + h] = load_w(x, src + h, dtype);
    }
    const int ldx = H + 64, ldi = I + 64;  // rows 64 B apart from a multiple of 1 KB
    xq.assign(static_cast<size_t>(m) * ldx, 128);
    const float xs = quantize_rows_u8(xa.data(), m, H, xq.data(), ldx, tmp, n_threads);
    acc1.assign(static_cast<size_t>(m) * 2 * I, 0);
    dot8_rows(xq.data(), ldx, m, H, w1q[e], rs1[e], 2 * I, acc1.data(), 2 * I, n_threads, use);
    const float m1 = dequant_mul(xs, s1[e]);
    inter.resize(static_cast<size_t>(m) * I);
    const int mi = m * I;
#pragma omp parallel for schedule(static) num_threads(n_threads)
    for (int ji = 0; ji < mi; ++ji) {
      const int j = ji / I, i = ji % I;
      const float g = static_cast<float>(acc1[(size_t)j * 2 * I + i]) * m1;
      const float u = static_cast<float>(acc1[(size_t)j * 2 * I + I + i]) * m1;
      inter[ji] = act_mul(act, g, u);
    }
    iq.assign(static_cast<size_t>(m) * ldi, 128);
    const float is = quantize_rows_u8(inter.data(), m, I, iq.data(), ldi, tmp, n_threads);
    acc2.assign(static_cast<size_t>(m) * H, 0);
    dot8_rows(iq.data(), ldi, m, I, w2q[e], rs2[e], H, acc2.data(), H, n_threads, use);
    const float m2 = dequant_mul(is, s2[e]);
    // one slot per (token, expert): every output element is written once here
#pragma omp parallel for schedule(static) num_threads(n_threads)
    for (int h = 0; h < H; ++h)
      for (int j = 0; j < m; ++j) {
        const float y = static_cast<float>(acc2[(size_t)j * H + h]) * m2;
        out[static_cast<size_t>(slot_tokens[s0 + j]) * H + h] += y * slot_weights[s0 + j];
      }
  }
  return 0;
}

const char* moe355_host_last_error(void) { return g_err.c_str(); }

int moe355_host_version(void) { return 102; }

int moe355_host_experts(const void* x, int T, int H, int I, int dtype, int n_experts,
                        const void* const* w1, const void* const* w2,
                        const int32_t* slot_offsets, const int32_t* slot_tokens,
                        const float* slot_weights, int act, int n_threads, float* out) {
  if (!x || !out || !slot_offsets || (n_experts > 0 && (!w1 || !w2 || !slot_tokens ||
                                                         !slot_weights)))
    return fail(MOE355_HOST_EINVAL, "null pointer argument");
  if (T < 0 || H <= 0 || I <= 0 || n_experts < 0)
    return fail(MOE355_HOST_EINVAL, "bad sizes");
  if (dtype != MOE355_HOST_F32 && dtype != MOE355_HOST_BF16 && dtype != MOE355_HOST_F16)
    return fail(MOE355_HOST_EINVAL, "dtype must be f32, bf16 or f16");
  if (act < 0 || act > 2) return fail(MOE355_HOST_EINVAL, "unknown activation code");
  if (!have_avx2()) return fail(MOE355_HOST_ECPU, "the host CPU lacks AVX2/FMA/F16C");
  if (slot_offsets[0] != 0) return fail(MOE355_HOST_EINVAL, "slot_offsets[0] must be 0");
  for (int e = 0; e < n_experts; ++e) {
    if (slot_offsets[e + 1] < slot_offsets[e])
      return fail(MOE355_HOST_EINVAL, "slot_offsets must be non-decreasing");
    if (!w1[e] || !w2[e]) return fail(MOE355_HOST_EINVAL, "null expert weight pointer");
  }
  const int n_slots = n_experts > 0 ? slot_offsets[n_experts] : 0;
  for (int s = 0; s < n_slots; ++s)
    if (slot_tokens[s] < 0 || slot_tokens[s] >= T)
      return fail(MOE355_HOST_EINVAL, "slot token index out of range");
  if (n_threads <= 0) n_threads = omp_get_max_threads();
  const Isa use = isa();
  const bool dp = use == kAvx512Bf16 && dtype == MOE355_HOST_BF16;

  std::vector<float> xa, gu, inter, y;
  std::vector<uint16_t> xa16, inter16;
  for (int e = 0; e < n_experts; ++e) {
    const int s0 = slot_offsets[e], m = slot_offsets[e + 1] - s0;
    if (m == 0) continue;
    // token rows padded by 64 bytes: rows n*4 bytes apart (n a multiple of
    // 1024, as H and I usually are) would all fall in the same L1 sets
    const int ldx = H + 16, ldi = I + 16, ldx16 = H + 32, ldi16 = I + 32;
    if (dp) {
      xa16.assign(static_cast<size_t>(m) * ldx16, 0);
      for (int j = 0; j < m; ++j)
        std::memcpy(&xa16[(size_t)j * ldx16],
                    static_cast<const uint16_t*>(x) + static_cast<size_t>(slot_tokens[s0 + j]) * H,
                    sizeof(uint16_t) * H);
    } else {
      xa.assign(static_cast<size_t>(m) * ldx, 0.0f);
      for (int j = 0; j < m; ++j) {
        const size_t src = static_cast<size_t>(slot_tokens[s0 + j]) * H;
        for (int h = 0; h < H; ++h) xa[(size_t)j * ldx + h] = load_w(x, src + h, dtype);
      }
    }
    // gate|up: [m, 2I], gate rows first
    gu.assign(static_cast<size_t>(m) * 2 * I, 0.0f);
    dot_rows(xa.data(), ldx, xa16.data(), ldx16, m, H, w1[e], dtype, 2 * I, gu.data(), 2 * I,
             n_threads, use);
    if (dp)
      inter16.assign(static_cast<size_t>(m) * ldi16, 0);
    else
      inter.assign(static_cast<size_t>(m) * ldi, 0.0f);
    const int mi = m * I;
#pragma omp parallel for schedule(static) num_threads(n_threads)
    for (int ji = 0; ji < mi; ++ji) {
      const int j = ji / I, i = ji % I;
      const float v = act_mul(act, gu[(size_t)j * 2 * I + i], gu[(size_t)j * 2 * I + I + i]);
      if (dp)
        inter16[(size_t)j * ldi16 + i] = f32_to_bf16(v);
      else
        inter[(size_t)j * ldi + i] = round_to_type(v, dtype);
    }
    // down: [m, H]
    y.assign(static_cast<size_t>(m) * H, 0.0f);
    dot_rows(inter.data(), ldi, inter16.data(), ldi16, m, I, w2[e], dtype, H, y.data(), H,
             n_threads, use);
#pragma omp parallel for schedule(static) num_threads(n_threads)
    for (int h = 0; h < H; ++h)
      for (int j = 0; j < m; ++j)
        out[static_cast<size_t>(slot_tokens[s0 + j]) * H + h] += slot_weights[s0 + j] * y[(size_t)j * H + h];
  }
  return 0;
}

}  // extern "C"
