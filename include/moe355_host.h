/* moe355_host.h — C ABI of libmoe355_host.so, the host-side half of the
 * CPU/GPU split MoE forward.
 *
 * Replaces the CPU half of the reference's split forward:
 *   reframework/moe/moe_layer.py:523-627  (FusedMoE._forward_split: misses
 *                                           computed on the CPU, summed with
 *                                           the GPU half)
 *   reframework/moe/fused.py:140-197      (fused_experts_cpu_int8)
 * The reference quantizes the host bank to int8 and multiplies with
 * torch._int_mm; this library multiplies the staged 16-bit (or fp32)
 * weights directly, with the same numerics as the device kernels: fp32
 * gate|up, the activated intermediate rounded once to the weight type, fp32
 * down projection, routing weight applied in fp32.
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

/* Version of this ABI (100). */
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

#ifdef __cplusplus
}
#endif

#endif /* MOE355_HOST_H */
