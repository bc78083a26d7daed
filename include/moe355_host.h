/* moe355_host.h — C ABI of libmoe355_host.so, the host-side half of the
 * CPU/GPU split MoE forward.
 *
 * Replaces the CPU half of the reference's split forward:
 *   reframework/moe/moe_layer.py:523-627  (FusedMoE._forward_split: misses
 *                                           computed on the CPU, summed with
 *                                           the GPU half)
 *   reframework/moe/fused.py:140-197      (fused_experts_cpu_int8)
 * The reference quantizes the host bank to int8 and multiplies with
 * torch._int_mm (moe355_host_experts_int8 restates that). moe355_host_experts
 * multiplies the staged 16-bit (or fp32) weights directly, with the same
 * numerics as the device kernels: fp32 gate|up, the activated intermediate
 * rounded once to the weight type, fp32 down projection, routing weight
 * applied in fp32.
 *
 * Host memory only (pinned or pageable), no GPU calls, no allocation visible
 * to the caller beyond per-call scratch. Thread-safe except for the
 * per-thread error string. Status: 0 ok, negative on a bad argument.
 */
#ifndef MOE355_HOST_H
#define MOE355_HOST_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MOE355_HOST_F32 0
#define MOE355_HOST_BF16 1
#define MOE355_HOST_F16 2

#define MOE355_HOST_EINVAL (-1)
#define MOE355_HOST_ECPU (-2)

/* Version of this ABI (102). */
int moe355_host_version(void);

/* Message of the last failed call on this thread. */
const char* moe355_host_last_error(void);

/* out[t, :] += sum over slots s of expert e routed from token t of
 *   w[s] * (act(x[t] W1g[e]^T) * (x[t] W1u[e]^T)) W2[e]^T
 * for the n_experts experts given.
 *   x            [T, H] in dtype (MOE355_HOST_*), row-major
 *   w1[e]        [2I, H] gate rows then up rows; w2[e] [H, I]; dtype as x
 *   slot_offsets [n_experts + 1]: expert e owns slots slot_offsets[e] ..
 *                slot_offsets[e+1]-1
 *   slot_tokens  token index of each slot; slot_weights its routing weight
 *   act          0 silu, 1 gelu (erf), 2 gelu (tanh)
 *   n_threads    <= 0: the OpenMP default
 *   out          [T, H] fp32, accumulated (the caller zeroes it)
 * Replaces fused_experts_cpu_int8 (reframework/moe/fused.py:140-197) with the
 * token index of each slot taken from its own (token, k) position. */
int moe355_host_experts(const void* x, int T, int H, int I, int dtype, int n_experts,
                        const void* const* w1, const void* const* w2,
                        const int32_t* slot_offsets, const int32_t* slot_tokens,
                        const float* slot_weights, int act, int n_threads, float* out);

/* Symmetric per-tensor int8 codes of a [rows, cols] weight in dtype:
 * amax = max |w|; amax <= 0 gives zero codes and *scale = 1; otherwise
 * *scale = amax / 127 (fp32) and q = clamp(round_half_even(w / scale), -127,
 * 127), the division in fp32. row_sums[r] = sum of row r's codes (the int8
 * expert call needs them). Replaces _sym_int8_quantize as called by
 * quantize_int8_host (reframework/moe/offload_cache.py:58-72, 386-407). */
int moe355_host_quantize_int8(const void* w, int rows, int cols, int dtype, int8_t* q,
                              float* scale, int32_t* row_sums, int n_threads);

/* row_sums[r] = sum of row r's codes of a [rows, cols] int8 matrix: the row
 * sums moe355_host_experts_int8 needs, for codes that did not come from
 * moe355_host_quantize_int8 (the int8 banks fused_experts_cpu_int8 is handed,
 * reframework/moe/fused.py:140-151, as packed by cpu_banks,
 * reframework/moe/offload_cache.py:409-434). */
int moe355_host_int8_row_sums(const int8_t* q, int rows, int cols, int32_t* row_sums,
                              int n_threads);

/* moe355_host_experts on int8 weights with the reference's numerics
 * (fused_experts_cpu_int8, reframework/moe/fused.py:140-197): per expert, the
 * token rows of its slots (x in dtype, widened to fp32) are quantized as one
 * block like the weights; gate|up is the exact integer product dequantized as
 * fp32(acc) * fp32(xs * s1[e]); act(g) * u in fp32; the [m, I] intermediate
 * block is quantized the same way; y = fp32(acc) * fp32(is * s2[e]), times the
 * slot's weight, added to out in fp32. w1q[e] [2I, H] and w2q[e] [H, I] are
 * codes with scales s1[e], s2[e] and row code sums rs1[e] [2I], rs2[e] [H]
 * from moe355_host_quantize_int8. Slots and out as moe355_host_experts (each
 * slot's own token, not the reference's i % M). H and I at most 65536 (the
 * integer sums stay in int32). */
int moe355_host_experts_int8(const void* x, int T, int H, int I, int dtype, int n_experts,
                             const int8_t* const* w1q, const int8_t* const* w2q, const float* s1,
                             const float* s2, const int32_t* const* rs1,
                             const int32_t* const* rs2, const int32_t* slot_offsets,
                             const int32_t* slot_tokens, const float* slot_weights, int act,
                             int n_threads, float* out);

#ifdef __cplusplus
}
#endif

#endif /* MOE355_HOST_H */
