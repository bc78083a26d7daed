/*
 * moe355 — C ABI of the MI355X (gfx950) MoE layer forward.
 *
 * One shared library, libmoe355.so. Every entry point:
 *   - takes raw device pointers, plain sizes and a hipStream_t (passed as void*);
 *   - is stream-ordered, performs no host synchronisation and allocates no device
 *     memory: scratch space is a caller-provided workspace whose size comes from
 *     moe355_make_plan();
 *   - returns 0 on success or a negative MOE355_E* status; moe355_last_error()
 *     gives a human-readable message for the calling thread.
 *
 * Layouts (all row-major, contiguous):
 *   x        [T, H]        tokens in the layer dtype
 *   gate     [E, H]        router weight (nn.Linear layout: out x in)
 *   w1[e]    [2I, H]       gate rows 0..I-1 followed by up rows I..2I-1
 *   w2[e]    [H, I]        down projection
 *   topk_w   [T, K] fp32   routing weights, slot (t,k) = t*K + k
 *   topk_ids [T, K] int32  (or int64 where a flag says so)
 *   out      [T, H]
 *
 * The reference implementation is pure PyTorch (reframework/moe/ package); each
 * declaration below names the reference code it replaces.
 */
#ifndef MOE355_H
#define MOE355_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* element types */
#define MOE355_F32 0
#define MOE355_BF16 1
#define MOE355_F16 2

/* gated activations, gate-first halves (reframework/layers/activation.py:15-59) */
#define MOE355_ACT_SILU 0
#define MOE355_ACT_GELU 1
#define MOE355_ACT_GELU_TANH 2

/* status codes */
#define MOE355_OK 0
#define MOE355_EINVAL (-1)       /* bad argument (null pointer, size, alignment) */
#define MOE355_EUNSUPPORTED (-2) /* shape or type the library does not handle */
#define MOE355_EWORKSPACE (-3)   /* workspace smaller than the plan requires */
#define MOE355_EHIP (-4)         /* a HIP runtime call failed */

/* Largest expert count accepted (pointer tables travel as kernel arguments). */
#define MOE355_MAX_EXPERTS 256

/* Kernel family chosen for the expert FFN. */
#define MOE355_PATH_MFMA_TILED 0 /* 256x256 bf16/f16 MFMA tiles, prefill-sized groups */
#define MOE355_PATH_MFMA_SKINNY 1 /* weight-streaming 16x16x32 MFMA, decode-sized groups */
#define MOE355_PATH_SIMT 2        /* fp32 FMA tiles: fp32 layers and unaligned shapes */
/* 3 is unused (a 256x64-tile family that no workload chose was removed) */
#define MOE355_PATH_MFMA_TILED128 4 /* the 256x256 kernel on 128-row token tiles, groups of ~128 rows */

/* Execution plan of one fused_experts call. Filled by moe355_make_plan() from
 * the shape alone (no device data), so every stage sees the same layout. */
typedef struct moe355_plan {
  int path;        /* MOE355_PATH_* */
  int tile_rows;   /* token rows per expert-FFN tile (tile-map granularity) */
  int max_tiles;   /* capacity of the tile map: upper bound of sum_e ceil(m_e/tile_rows) */
  int down_splits; /* K-splits of the down projection; y holds one fp32 partial per split */
  int rows;        /* T*K routed slots */
  int n_blocks;    /* permute blocks (1024 slots each) */
  int T, H, I, E, K, dtype;
  size_t workspace_bytes;
  /* byte offsets into the workspace */
  size_t off_block_counts; /* int32 [n_blocks, E] */
  size_t off_offsets;      /* int32 [E+1]    expert_offsets: rows of expert e are [off[e], off[e+1]) */
  size_t off_slot_to_row;  /* int32 [T*K]    permuted row of slot (t,k), -1 when dropped */
  size_t off_row_src;      /* int32 [T*K]    source token of each permuted row */
  size_t off_tile_map;     /* int32 [2 + 2*max_tiles]: count, tile_rows, then (expert, first_row)
                              pairs; an expert's tiles are consecutive and lie its tile height
                              apart (tile_rows, or on 256-row maps its rows over its tiles rounded
                              up to 32); experts in any order (the permute: largest, smallest,
                              second largest, ..) */
  size_t off_inter;        /* dtype [T*K, I] silu(gate)*up per permuted row */
  size_t off_y;            /* fp32  [down_splits, T*K, H] down-projection partials; for the
                              tiled paths with down_splits == 1, dtype [T*K, H] (rounded to
                              the layer dtype, as the reference's bf16 matmul returns it) */
  size_t off_part;         /* fp32 256x256 partial tiles of the tiled down projection's K-split
                              last-round items, up to one per CU (empty for the other paths) */
} moe355_plan;

/* Library version (major*10000 + minor*100 + patch). */
int moe355_version(void);

/* Message describing the last failure on the calling thread ("" if none). */
const char* moe355_last_error(void);

/*
 * Router GEMM + softmax + top-k in one kernel.
 * Replaces FusedMoE.route (reframework/moe/moe_layer.py:320-344): the router
 * F.linear at :324 followed by torch_fused_topk (reframework/moe/fused.py:32-46).
 *   logits[t,e] = sum_h x[t,h]*gate[e,h] accumulated in fp32; if round_logits,
 *                 rounded to `dtype` (the reference's F.linear output is in the
 *                 model dtype); then + bias[e] when bias != NULL.
 *   p = softmax(logits); ids = the K largest logits, descending, ties -> lower id;
 *   w = p[ids], divided by sum(w) when renormalize.
 * entropy_k_min > 0 enables the entropy-adaptive branch of route() (:326-342):
 *   k_dyn = clamp(rint(k_min + (K-k_min)*Hnorm(p)), k_min, K); weights past k_dyn
 *   are zeroed and the rest renormalised (ids are kept).
 * logits_out [T,E] fp32 is optional (NULL to skip). Given, it also serves as
 * the router's scratch: below 256 tokens with more than 16 experts the logits
 * are computed by (token, 8-expert) workgroups into it and selected by a
 * second launch (the ids then follow those logits bit for bit, as always).
 */
int moe355_router_topk(const void* x, const void* gate, const float* bias, int T, int H, int E,
                       int K, int dtype, int renormalize, int round_logits, int entropy_k_min,
                       float* logits_out, float* topk_w, int32_t* topk_ids, void* stream);

/*
 * moe355_router_topk writing token t's K weights and ids at row t of [T, out_ld]
 * arrays (out_ld >= K; columns K.. are left untouched). The same replacement of
 * FusedMoE.route (reframework/moe/moe_layer.py:320-344); the stride lets the
 * routed ids land beside constant columns, e.g. the always-on shared experts
 * folded in as extra experts with weight 1 (which the reference does not have).
 */
int moe355_router_topk_ld(const void* x, const void* gate, const float* bias, int T, int H, int E,
                          int K, int dtype, int renormalize, int round_logits, int entropy_k_min,
                          float* logits_out, float* topk_w, int32_t* topk_ids, int out_ld,
                          void* stream);

/*
 * residual_out = x + residual (rounded to `dtype`; residual_out may alias x or
 * residual), then normed = residual_out / sqrt(mean(residual_out^2) + eps) *
 * weight (+ bias), in fp32, rounded once. With residual == NULL: normed =
 * rmsnorm(x) and residual_out is unused (x may alias normed_out). weight/bias
 * are [H] in weight_dtype; bias may be NULL.
 * Replaces RMSNorm._forward / forward_add_residual
 * (reframework/layers/norm.py:27-53), the step before the MoE block at
 * reframework/models/base.py:135.
 */
int moe355_add_rmsnorm(const void* x, const void* residual, void* residual_out,
                       const void* weight, const void* bias, int weight_dtype, float eps, int T,
                       int H, int dtype, void* normed_out, void* stream);

/*
 * moe355_add_rmsnorm followed by moe355_router_topk on the normed rows, in one
 * call on one stream: post_attention_layernorm.forward_add_residual + route
 * (reframework/models/base.py:135-136, moe/moe_layer.py:320-344). For bf16/f16
 * with H <= 8192 (a multiple of 8), T * E <= 8192 and E <= 16 (E <= 64 when
 * logits_out is NULL) one kernel does both: the normed rows (written to
 * normed_out, bit for bit moe355_add_rmsnorm's) stay in registers for the
 * router's dot products. The router's fp32 sums then run in another order than
 * moe355_router_topk's, so a logit may round to the neighbouring bf16/f16 value.
 * logits_out ([T,E] fp32, the logits top-k ranked) may be NULL.
 */
int moe355_add_rmsnorm_router_topk(const void* x, const void* residual, void* residual_out,
                                   const void* norm_weight, const void* norm_bias,
                                   int weight_dtype, float eps,
                                   const void* gate, const float* router_bias, int T, int H, int E,
                                   int K, int dtype, int renormalize, int round_logits,
                                   void* normed_out, float* logits_out, float* topk_w,
                                   int32_t* topk_ids, void* stream);

/*
 * softmax -> top-k -> renormalise on given fp32 logits.
 * Replaces torch_fused_topk (reframework/moe/fused.py:32-46). Selection is on
 * the logits (monotone with the softmax), ties -> lower expert id.
 */
int moe355_topk_from_logits(const float* logits, int T, int E, int K, int renormalize,
                            float* topk_w, int32_t* topk_ids, void* stream);

/* Fill `plan` for a fused_experts call of this shape. Host-side; reads the
 * current device's CU count (256 without a device) to choose the down
 * projection's K-split, and launches nothing. The kernel family follows the
 * average rows per active expert (T*K / min(T*K, E)): up to 10 skinny, up to
 * 104 the tiled kernel on 128-row tiles, above it 256-row tiles; fp32 and
 * shapes the MFMA kernels do not tile take the SIMT family. */
int moe355_make_plan(int T, int H, int I, int E, int K, int dtype, moe355_plan* plan);

/* moe355_make_plan with the kernel family forced (`path` = MOE355_PATH_*, or -1
 * for the automatic choice); MOE355_EUNSUPPORTED if that family cannot run the
 * shape. No counterpart in the reference: for tests and tuning, so that every
 * family can be checked at any shape. */
int moe355_make_plan_path(int T, int H, int I, int E, int K, int dtype, int path,
                          moe355_plan* plan);

/*
 * Stable counting sort of the routed slots by expert.
 * Replaces the grouping of fused_experts (reframework/moe/fused.py:70-80):
 * experts in ascending id, slots in ascending (t,k) order within an expert.
 * expert_map (host array, map_len entries, may be NULL) renames ids before the
 * sort: local = expert_map[id]; a negative entry, or an id outside [0,map_len)
 * (without a map: outside [0,E)), drops the slot. This is the global->local
 * remap and the slot truncation of FusedMoE.forward (moe_layer.py:477-511).
 * Writes block_counts, offsets, slot_to_row, row_src and tile_map.
 */
int moe355_permute(const moe355_plan* plan, const void* topk_ids, int ids_int64,
                   const int32_t* expert_map, int map_len, void* workspace, void* stream);

/*
 * Grouped gate|up projection with the gated activation fused in the epilogue:
 * inter[r, :] = act(x[src(r)] . w1[e][:I]^T) * (x[src(r)] . w1[e][I:]^T) for
 * every permuted row r of expert e. Replaces `x @ w1[e].t()` and
 * gated_act_and_mul (reframework/moe/fused.py:80-82). w1 is a host array of
 * E device pointers (per-expert banks; no stacking copy).
 */
int moe355_gate_up(const moe355_plan* plan, const void* x, const void* const* w1, int act,
                   void* workspace, void* stream);

/*
 * Grouped down projection: y[s, r, :] = partial (split s) of inter[r] . w2[e]^T.
 * Replaces `inter @ w2[e].t()` (reframework/moe/fused.py:83).
 */
int moe355_down(const moe355_plan* plan, const void* const* w2, void* workspace, void* stream);

/*
 * Weighted combine back to token order:
 *   out[t] = sum_k topk_w[t,k] * sum_s y[s, slot_to_row[t*K+k]]   (dropped slots skipped)
 * accumulated in fp32, k ascending, y read in the format the plan's down
 * projection writes (see off_y). Replaces `y * w; out.index_add_(0, tok, y)`
 * (reframework/moe/fused.py:84-86). With accumulate_f32 = 0, out has the plan
 * dtype and is overwritten; with 1, out is fp32 and the sum is added to it (the
 * fp32 accumulator of FusedMoE._forward_streaming, moe_layer.py:370,415).
 */
int moe355_combine(const moe355_plan* plan, const float* topk_w, void* out, int accumulate_f32,
                   void* workspace, void* stream);

/*
 * The whole routed-expert computation: permute, gate_up, down, combine.
 * Replaces fused_experts (reframework/moe/fused.py:49-87); x, w1 and w2 share
 * `dtype`. workspace must hold plan.workspace_bytes (moe355_make_plan).
 * A slot whose topk_w is exactly 0 is dropped like an unmapped one: it would
 * add 0 * y. The reference's expert-parallel layer zeroes the weights of
 * other ranks' experts and maps them to local row 0 (parallel/ep.py:137-143);
 * those slots then cost nothing here instead of piling onto expert 0.
 */
int moe355_fused_experts(const void* x, const void* const* w1, const void* const* w2,
                         const float* topk_w, const void* topk_ids, int ids_int64,
                         const int32_t* expert_map, int map_len, int T, int H, int I, int E,
                         int K, int dtype, int act, void* out, int accumulate_f32,
                         void* workspace, size_t workspace_bytes, void* stream);

/* Size of the library's static scratch (moe355_fused_experts_static). */
#define MOE355_STATIC_SCRATCH_BYTES (64u << 20)

/*
 * moe355_fused_experts without a workspace argument: scratch comes from a
 * static device array of MOE355_STATIC_SCRATCH_BYTES inside the library (one
 * per device, held until the process ends), so the call allocates nothing
 * and needs no buffer from the caller.
 * No counterpart in the reference. It is for callers that cannot allocate
 * device memory: code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc.
 * Limits: a shape whose plan needs more than MOE355_STATIC_SCRATCH_BYTES
 * fails with MOE355_EWORKSPACE before launching anything (the tiled paths
 * first drop their down-projection partial tiles, running that projection's
 * last round whole). The calling thread's current device must be the device
 * of `stream`. Every call on one device shares that device's array: calls
 * that overlap on one device (other streams, other threads) race and must
 * be serialised by the caller. Nothing in the array needs to start zeroed.
 */
int moe355_fused_experts_static(const void* x, const void* const* w1, const void* const* w2,
                                const float* topk_w, const void* topk_ids, int ids_int64,
                                const int32_t* expert_map, int map_len, int T, int H, int I,
                                int E, int K, int dtype, int act, void* out, int accumulate_f32,
                                void* stream);

/*
 * Cast an fp32 [n] buffer to `dtype` (the final cast of the streaming path,
 * reframework/moe/moe_layer.py:418).
 */
int moe355_cast_f32(const float* src, void* dst, size_t n, int dtype, void* stream);

/*
 * Zero-copy staging for the CPU/GPU split forward. The reference's split moves
 * the step's routing and hidden states to the host with synchronous copies
 * (`topk_ids.reshape(-1).tolist()`, reframework/moe/moe_layer.py:550-551;
 * `hidden_states.detach().cpu()`, reframework/moe/fused.py:175) and the host
 * half back with `cpu_out.to(dev)` (moe_layer.py:597). On MI355X those small
 * transfers would queue on the DMA engines behind the 352 MB expert copies
 * the split keeps in flight, so a kernel on the compute stream moves them
 * through mapped pinned host memory instead.
 *
 * moe355_host_staging_alloc: `bytes` of mapped, coherent pinned host memory
 * (hipHostMalloc), readable and writable by kernels. Free with
 * moe355_host_staging_free once no queued kernel uses it.
 */
int moe355_host_staging_alloc(size_t bytes, void** host_ptr);
int moe355_host_staging_free(void* host_ptr);

/*
 * Copy `bytes` of device memory at `src` into staging memory at `host_dst`
 * (any address inside a moe355_host_staging_alloc buffer, or other mapped
 * pinned memory) with a kernel on `stream`; both 16-byte aligned. The host
 * reads the bytes after waiting for an event recorded behind the call.
 */
int moe355_copy_to_host(void* host_dst, const void* src, size_t bytes, void* stream);

/*
 * moe355_copy_to_host for n <= 4 regions in one kernel launch: src[k]
 * (device, bytes[k]) to host_dst + dst_offsets[k], all 16-byte aligned. The
 * split forward hands a step's routing ids, weights and hidden states to the
 * host this way (the .tolist() / .cpu() of moe_layer.py:523-627), paying one
 * launch and one release of the writes to host memory instead of three.
 */
int moe355_copy_to_host_multi(void* host_dst, int n, const void* const* src,
                              const size_t* dst_offsets, const size_t* bytes, void* stream);

/*
 * out[i] = (dtype) (acc[i] + host_src[i]) for i < n, reading host_src
 * (fp32 in mapped pinned memory, written by the host before the call) from
 * the kernel: the merge `out.float() + cpu_out.to(dev)` then `.to(x2.dtype)`
 * of reframework/moe/moe_layer.py:597-598. n a multiple of 4; acc, host_src
 * 16-byte aligned; acc is fp32 device memory, out [n] of `dtype`.
 */
int moe355_merge_host_f32(const float* acc, const float* host_src, size_t n, int dtype, void* out,
                          void* stream);

/*
 * Host -> HBM expert copy on `stream` (a side stream), asynchronous when `src`
 * is pinned. Replaces ExpertOffloadCache._fill's `.to(device, non_blocking)`
 * (reframework/moe/offload_cache.py:645-652). Completion is observed with an
 * event the caller records on the same stream.
 */
int moe355_h2d_async(void* dst, const void* src, size_t bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MOE355_H */
