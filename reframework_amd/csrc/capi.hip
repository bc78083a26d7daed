// The extern "C" boundary of libmoe355.so: argument checks, the execution
// plan, and dispatch to the kernel launchers. Declarations and their reference
// counterparts are in include/moe355.h.
#include <algorithm>
#include <climits>
#include <cstdarg>
#include <cstdio>
#include <cstring>

#include <mutex>

#include "common.h"

using namespace moe355;

// Scratch of moe355_fused_experts_static: the workspace of callers that cannot
// allocate. Each device that loads the library holds its own copy until the
// process ends; see static_scratch for how host code reaches it.
static __device__ __align__(256) unsigned char scratch[MOE355_STATIC_SCRATCH_BYTES];

namespace {

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int check_hip(hipError_t e, const char* what) {
  if (e == hipSuccess) return MOE355_OK;
  return fail(MOE355_EHIP, "%s: %s", what, hipGetErrorString(e));
}

constexpr int kMaxDevices = 64;

size_t align256(size_t v) { return (v + 255) & ~static_cast<size_t>(255); }

bool valid_dtype(int d) { return d == MOE355_F32 || d == MOE355_BF16 || d == MOE355_F16; }

int elem_size(int d) { return d == MOE355_F32 ? 4 : 2; }

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

hipStream_t as_stream(void* s) { return static_cast<hipStream_t>(s); }

template <typename T>
T* at(void* ws, size_t off) {
  return reinterpret_cast<T*>(static_cast<char*>(ws) + off);
}

int check_plan(const moe355_plan* p) {
  if (!p) return fail(MOE355_EINVAL, "plan is NULL");
  if (p->E < 1 || p->E > MOE355_MAX_EXPERTS || p->K < 1 || p->K > p->E || !valid_dtype(p->dtype) ||
      p->path < 0 || p->path > MOE355_PATH_MFMA_TILED128 || p->path == 3 ||
      p->rows != p->T * p->K)
    return fail(MOE355_EINVAL, "plan is not one filled by moe355_make_plan");
  return MOE355_OK;
}

int check_banks(const moe355_plan* p, const void* const* w, const char* name) {
  if (!w) return fail(MOE355_EINVAL, "%s pointer table is NULL", name);
  for (int e = 0; e < p->E; ++e) {
    if (!w[e]) return fail(MOE355_EINVAL, "%s[%d] is NULL", name, e);
    if (p->path != MOE355_PATH_SIMT && !aligned16(w[e]))
      return fail(MOE355_EINVAL, "%s[%d] is not 16-byte aligned", name, e);
  }
  return MOE355_OK;
}

}  // namespace

namespace moe355 {

int device_cu_count() {
  static int cached[kMaxDevices] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    (void)hipGetLastError();
    return 256;
  }
  if (cached[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) {
      (void)hipGetLastError();
      n = 256;
    }
    cached[dev] = n;
  }
  return cached[dev];
}

}  // namespace moe355

extern "C" {

int moe355_version(void) { return 101; }

const char* moe355_last_error(void) { return g_err; }

int moe355_make_plan(int T, int H, int I, int E, int K, int dtype, moe355_plan* p) {
  return moe355_make_plan_path(T, H, I, E, K, dtype, -1, p);
}

int moe355_make_plan_path(int T, int H, int I, int E, int K, int dtype, int path,
                          moe355_plan* p) {
  if (!p) return fail(MOE355_EINVAL, "plan is NULL");
  if (path < -1 || path > MOE355_PATH_MFMA_TILED128 || path == 3)
    return fail(MOE355_EINVAL, "unknown path %d", path);
  if (T < 0 || H <= 0 || I <= 0) return fail(MOE355_EINVAL, "bad sizes T=%d H=%d I=%d", T, H, I);
  if (E < 1 || E > MOE355_MAX_EXPERTS)
    return fail(MOE355_EUNSUPPORTED, "E=%d outside [1, %d]", E, MOE355_MAX_EXPERTS);
  if (K < 1 || K > E) return fail(MOE355_EINVAL, "top-k K=%d outside [1, E=%d]", K, E);
  if (!valid_dtype(dtype)) return fail(MOE355_EINVAL, "unknown dtype %d", dtype);
  const int esz = elem_size(dtype);
  const int vec = 16 / esz;
  if (H % vec || I % vec)
    return fail(MOE355_EUNSUPPORTED, "H=%d and I=%d must be multiples of %d", H, I, vec);
  const long long R = static_cast<long long>(T) * K;
  if (R > INT_MAX / 2) return fail(MOE355_EUNSUPPORTED, "T*K=%lld too large", R);

  std::memset(p, 0, sizeof(*p));
  p->T = T; p->H = H; p->I = I; p->E = E; p->K = K; p->dtype = dtype;
  p->rows = static_cast<int>(R);
  p->n_blocks = R <= kPermuteSingleMax ? 1 : static_cast<int>((R + kPermuteChunk - 1) / kPermuteChunk);
  const int act_e = static_cast<int>(R < E ? (R > 0 ? R : 1) : E);
  const long long avg = R / act_e;

  const bool mfma = dtype != MOE355_F32;
  // Token rows are addressed by 32-bit byte offsets whose bit 31 marks tile
  // padding (loaded as zeros), so x must stay below 2 GB; weight offsets are
  // 32-bit too.
  const bool tiled_ok = mfma && H % 256 == 0 && I % 128 == 0 &&
                        static_cast<long long>(T) * H * esz < (1ll << 31) &&
                        2ll * I * H * esz < (1ll << 32);
  const bool skinny_ok = mfma && H % 128 == 0 && I % 128 == 0;
  if (path < 0) {
    // Average rows per active expert decide (measured layer times, Mixtral,
    // Phi-3.5 and fine-grained shapes): weight streaming with 16-token tiles up
    // to 10 rows (beyond that each 16-row tile re-streams the weights), the
    // 256-row kernel on 128-row tiles up to 104 rows (Mixtral 64 and 256
    // tokens: 0.55 and 0.59 ms against 0.56 and 0.65 with 256-row tiles;
    // fine-grained 512 tokens 0.31 against 0.32), 256-row tiles above
    // (Mixtral 512 tokens: 0.67 against 0.68 ms).
    path = tiled_ok && avg > 104  ? MOE355_PATH_MFMA_TILED
           : tiled_ok && avg > 10 ? MOE355_PATH_MFMA_TILED128
           : skinny_ok            ? MOE355_PATH_MFMA_SKINNY
                                  : MOE355_PATH_SIMT;
  } else if (((path == MOE355_PATH_MFMA_TILED || path == MOE355_PATH_MFMA_TILED128) &&
              !tiled_ok) ||
             (path == MOE355_PATH_MFMA_SKINNY && !skinny_ok)) {
    return fail(MOE355_EUNSUPPORTED, "path %d cannot run dtype %d with H=%d I=%d T=%d", path,
                dtype, H, I, T);
  }
  p->path = path;
  const bool tiled = path == MOE355_PATH_MFMA_TILED || path == MOE355_PATH_MFMA_TILED128;
  p->tile_rows = path == MOE355_PATH_MFMA_TILED      ? 256
                 : path == MOE355_PATH_MFMA_TILED128 ? 128
                 : path == MOE355_PATH_MFMA_SKINNY   ? 16
                                                     : 64;
  p->max_tiles = R > 0 ? static_cast<int>((R + static_cast<long long>(act_e) * (p->tile_rows - 1)) /
                                          p->tile_rows)
                       : 0;
  p->down_splits = 1;
  if (tiled) {
    // The persistent down kernels run (H/256 weight tiles x token tiles x
    // splits) work items of I/(32*splits) 32-k steps on one workgroup per CU.
    // Pick the split that minimises the busiest CU's step count, charging each
    // extra split its fp32 partial plane (written once, read by the combine)
    // at ~1.8e-6 steps per element; ties keep fewer splits. The kernel cuts a
    // partly idle last round along K (work_split, same rule), so its last
    // round costs what that cut leaves. Each split must be a whole number of
    // 64-k pipeline steps. Token tiles are estimated per active expert as its
    // average rows over the tile height plus half a tile for the ragged end,
    // at least one (Mixtral 4096 tokens: 36, as routed;
    // 128 and 256 tokens on 128-row tiles: 8): max_tiles is a worst case, and
    // sizing the split by it cut layers finer than their real tile count pays
    // for (Mixtral 256, 512 and 1024 tokens: down 0.201, 0.225 and 0.318 ms
    // with the worst case, 0.183, 0.204 and 0.283 with the estimate).
    const double est_tiles =
        std::min(static_cast<double>(p->max_tiles),
                 act_e * std::max(1.0, static_cast<double>(R) / act_e / p->tile_rows + 0.5));
    const long long items =
        static_cast<long long>(H / 256) * static_cast<long long>(est_tiles + 0.5);
    const int cus = moe355::device_cu_count();
    double best = 0.0;
    for (int s = 1; s <= 8 && (I / 64) % s == 0; s *= 2) {
      const long long n = items * s, full = n / cus, tail = n % cus;
      const double per_item = static_cast<double>(I / 32 / s);
      double last = tail ? per_item : 0.0;
      if (full > 0 && tail > 0) {
        const int nk = I / 64 / s;
        for (long long st = 2; st <= 16 && st * tail <= cus && nk % st == 0; st *= 2)
          last = std::min(last, 2.0 * (static_cast<double>(nk) / st + st * tail / 14.0));
      }
      const double cost = static_cast<double>(full) * per_item + last +
                          (s - 1) * static_cast<double>(R) * H * 1.8e-6;
      if (s == 1 || cost < 0.97 * best) {
        best = cost;
        p->down_splits = s;
      }
    }
  } else if (p->path == MOE355_PATH_MFMA_SKINNY) {
    // Spread the down projection (H/16 row groups per tile) over >= 8192 waves,
    // at most 8 splits (Mixtral shape: 4 splits instead of 2 at 4 and 16
    // tokens, down 98 -> 91 and 140 -> 133 us; 16 splits at one token are
    // 2 us slower than 8); each split covers a multiple of the kernel's
    // 128-element k step.
    const long long waves = static_cast<long long>(H / 16) * (p->max_tiles > 0 ? p->max_tiles : 1);
    int s = 1;
    while (s < 8 && waves * s < 8192 && (I / 128) % (2 * s) == 0) s *= 2;
    p->down_splits = s;
  }

  size_t off = 0;
  p->off_block_counts = off; off = align256(off + static_cast<size_t>(p->n_blocks) * E * 4);
  p->off_offsets = off;      off = align256(off + static_cast<size_t>(E + 1) * 4);
  p->off_slot_to_row = off;  off = align256(off + static_cast<size_t>(R) * 4);
  p->off_row_src = off;      off = align256(off + static_cast<size_t>(R) * 4);
  p->off_tile_map = off;     off = align256(off + static_cast<size_t>(2 + 2 * p->max_tiles) * 4);
  p->off_inter = off;        off = align256(off + static_cast<size_t>(R) * I * esz);
  p->off_y = off;            off = align256(off + static_cast<size_t>(p->down_splits) * R * H * 4);
  p->off_part = off;
  if (tiled) {
    // One 256 KB partial tile per CU: the tiled kernels cut the items of a
    // last, partly idle round along K over the idle CUs (at most one unit per
    // CU). gate_up also has the y region before it, free until the down
    // projection.
    off = align256(off + static_cast<size_t>(moe355::device_cu_count()) * 256 * 256 * 4);
  }
  p->workspace_bytes = off;
  return MOE355_OK;
}

int moe355_router_topk(const void* x, const void* gate, const float* bias, int T, int H, int E,
                       int K, int dtype, int renormalize, int round_logits, int entropy_k_min,
                       float* logits_out, float* topk_w, int32_t* topk_ids, void* stream) {
  return moe355_router_topk_ld(x, gate, bias, T, H, E, K, dtype, renormalize, round_logits,
                               entropy_k_min, logits_out, topk_w, topk_ids, K, stream);
}

int moe355_router_topk_ld(const void* x, const void* gate, const float* bias, int T, int H, int E,
                          int K, int dtype, int renormalize, int round_logits, int entropy_k_min,
                          float* logits_out, float* topk_w, int32_t* topk_ids, int out_ld,
                          void* stream) {
  if (T < 0 || H <= 0) return fail(MOE355_EINVAL, "bad sizes T=%d H=%d", T, H);
  if (E < 1 || E > MOE355_MAX_EXPERTS)
    return fail(MOE355_EUNSUPPORTED, "E=%d outside [1, %d]", E, MOE355_MAX_EXPERTS);
  if (K < 1 || K > E) return fail(MOE355_EINVAL, "top-k K=%d outside [1, E=%d]", K, E);
  if (!valid_dtype(dtype)) return fail(MOE355_EINVAL, "unknown dtype %d", dtype);
  if (entropy_k_min < 0 || entropy_k_min > K)
    return fail(MOE355_EINVAL, "entropy_k_min=%d outside [0, K=%d]", entropy_k_min, K);
  if (out_ld < K) return fail(MOE355_EINVAL, "output row stride %d < K=%d", out_ld, K);
  const int vec = 16 / elem_size(dtype);
  if (H % vec) return fail(MOE355_EUNSUPPORTED, "router needs H %% %d == 0", vec);
  if (T == 0) return MOE355_OK;
  if (!x || !gate || !topk_w || !topk_ids) return fail(MOE355_EINVAL, "NULL tensor argument");
  if (!aligned16(x) || !aligned16(gate)) return fail(MOE355_EINVAL, "x/gate not 16-byte aligned");
  RouterArgs a{};
  a.x = x; a.gate = gate; a.bias = bias; a.logits_in = nullptr; a.logits_out = logits_out;
  a.topk_w = topk_w; a.topk_ids = topk_ids;
  a.T = T; a.H = H; a.E = E; a.K = K;
  a.renormalize = renormalize != 0; a.round_logits = round_logits != 0;
  a.entropy_k_min = entropy_k_min; a.out_ld = out_ld;
  return check_hip(launch_router(a, dtype, as_stream(stream)), "router_topk launch");
}

int moe355_add_rmsnorm(const void* x, const void* residual, void* residual_out,
                       const void* weight, const void* bias, int weight_dtype, float eps, int T,
                       int H, int dtype, void* normed_out, void* stream) {
  if (T < 0 || H <= 0) return fail(MOE355_EINVAL, "bad sizes T=%d H=%d", T, H);
  if (!valid_dtype(dtype) || !valid_dtype(weight_dtype))
    return fail(MOE355_EINVAL, "unknown dtype %d / weight dtype %d", dtype, weight_dtype);
  const int vec = 16 / elem_size(dtype);
  if (H % vec || H > norm_max_hidden(dtype))
    return fail(MOE355_EUNSUPPORTED, "norm needs H %% %d == 0 and H <= %d", vec,
                norm_max_hidden(dtype));
  if (!(eps >= 0.0f)) return fail(MOE355_EINVAL, "eps must be >= 0");
  if (T == 0) return MOE355_OK;
  if (!x || !weight || !normed_out) return fail(MOE355_EINVAL, "NULL tensor argument");
  if (residual && !residual_out) return fail(MOE355_EINVAL, "residual given without residual_out");
  if (!aligned16(x) || !aligned16(normed_out) || (residual && !aligned16(residual)) ||
      (residual && !aligned16(residual_out)))
    return fail(MOE355_EINVAL, "x/residual/out not 16-byte aligned");
  if (!aligned16(weight) || (bias && !aligned16(bias)))
    return fail(MOE355_EINVAL, "norm weight/bias not 16-byte aligned");
  NormArgs a{};
  a.x = x; a.residual = residual; a.residual_out = residual_out; a.weight = weight;
  a.bias = bias; a.out = normed_out;
  a.T = T; a.H = H; a.weight_dtype = weight_dtype; a.eps = eps;
  return check_hip(launch_add_rmsnorm(a, dtype, as_stream(stream)), "add_rmsnorm launch");
}

int moe355_add_rmsnorm_router_topk(const void* x, const void* residual, void* residual_out,
                                   const void* norm_weight, const void* norm_bias,
                                   int weight_dtype, float eps,
                                   const void* gate, const float* router_bias, int T, int H, int E,
                                   int K, int dtype, int renormalize, int round_logits,
                                   void* normed_out, float* logits_out, float* topk_w,
                                   int32_t* topk_ids, void* stream) {
  const bool mfma = !norm_router_fusable(T, H, E, dtype, logits_out != nullptr) &&
                    norm_router_mfma_fusable(T, H, E, K, dtype);
  if (!mfma && !norm_router_fusable(T, H, E, dtype, logits_out != nullptr)) {
    int rc = moe355_add_rmsnorm(x, residual, residual_out, norm_weight, norm_bias, weight_dtype,
                                eps, T, H, dtype, normed_out, stream);
    if (rc) return rc;
    return moe355_router_topk_ld(normed_out, gate, router_bias, T, H, E, K, dtype, renormalize,
                                 round_logits, 0, logits_out, topk_w, topk_ids, K, stream);
  }
  // The arguments both halves would check, then one launch.
  if (T < 0 || H <= 0) return fail(MOE355_EINVAL, "bad sizes T=%d H=%d", T, H);
  if (!valid_dtype(weight_dtype)) return fail(MOE355_EINVAL, "unknown weight dtype %d", weight_dtype);
  if (K < 1 || K > E) return fail(MOE355_EINVAL, "top-k K=%d outside [1, E=%d]", K, E);
  if (!(eps >= 0.0f)) return fail(MOE355_EINVAL, "eps must be >= 0");
  if (T == 0) return MOE355_OK;
  if (!x || !norm_weight || !normed_out || !gate || !topk_w || !topk_ids)
    return fail(MOE355_EINVAL, "NULL tensor argument");
  if (residual && !residual_out) return fail(MOE355_EINVAL, "residual given without residual_out");
  if (!aligned16(x) || !aligned16(normed_out) || (residual && !aligned16(residual)) ||
      (residual && !aligned16(residual_out)) || !aligned16(gate))
    return fail(MOE355_EINVAL, "x/residual/out/gate not 16-byte aligned");
  if (!aligned16(norm_weight) || (norm_bias && !aligned16(norm_bias)))
    return fail(MOE355_EINVAL, "norm weight/bias not 16-byte aligned");
  NormArgs na{};
  na.x = x; na.residual = residual; na.residual_out = residual_out; na.weight = norm_weight;
  na.bias = norm_bias; na.out = normed_out;
  na.T = T; na.H = H; na.weight_dtype = weight_dtype; na.eps = eps;
  RouterArgs ra{};
  ra.x = normed_out; ra.gate = gate; ra.bias = router_bias; ra.logits_out = logits_out;
  ra.topk_w = topk_w; ra.topk_ids = topk_ids;
  ra.T = T; ra.H = H; ra.E = E; ra.K = K;
  ra.renormalize = renormalize != 0; ra.round_logits = round_logits != 0;
  ra.entropy_k_min = 0; ra.out_ld = K;
  if (mfma)
    return check_hip(launch_add_rmsnorm_router_mfma(na, ra, dtype, as_stream(stream)),
                     "add_rmsnorm_router_mfma launch");
  return check_hip(launch_add_rmsnorm_router(na, ra, dtype, as_stream(stream)),
                   "add_rmsnorm_router launch");
}

int moe355_topk_from_logits(const float* logits, int T, int E, int K, int renormalize,
                            float* topk_w, int32_t* topk_ids, void* stream) {
  if (T < 0) return fail(MOE355_EINVAL, "bad T=%d", T);
  if (E < 1 || E > MOE355_MAX_EXPERTS)
    return fail(MOE355_EUNSUPPORTED, "E=%d outside [1, %d]", E, MOE355_MAX_EXPERTS);
  if (K < 1 || K > E) return fail(MOE355_EINVAL, "top-k K=%d outside [1, E=%d]", K, E);
  if (T == 0) return MOE355_OK;
  if (!logits || !topk_w || !topk_ids) return fail(MOE355_EINVAL, "NULL tensor argument");
  RouterArgs a{};
  a.logits_in = logits; a.topk_w = topk_w; a.topk_ids = topk_ids;
  a.T = T; a.E = E; a.K = K; a.renormalize = renormalize != 0; a.out_ld = K;
  return check_hip(launch_topk_from_logits(a, as_stream(stream)), "topk_from_logits launch");
}

}  // extern "C"

namespace {

// Whether the full-tile kernels multiply only the token blocks each item's
// rows reach and rotate their XCD slots (the kRagged instance of
// ffn_tiled16_kernel) instead of the blocks of each expert's tile height:
// where experts hold on average two 256-row tiles or fewer (Mixtral 2048
// tokens gate_up 831 -> 822 us, fine-grained 4096 tokens 319 -> 314 us,
// Phi-3.5 2048 tokens 507 -> 504 us); at more rows per expert the uneven items
// cost about what they save (Mixtral 4096 tokens 1464 -> 1470 us).
bool ragged_tiles(const moe355_plan* p) {
  const long long act = std::min<long long>(p->E, p->rows);
  return act > 0 && p->rows / act <= 2 * 256;
}

// Checks the permute's arguments and fills its kernel arguments (the caller
// has checked the plan and that it has rows).
int permute_args(const moe355_plan* p, const void* topk_ids, int ids_int64,
                 const int32_t* expert_map, int map_len, void* workspace, PermuteArgs* a,
                 const float* topk_w = nullptr) {
  if (map_len < 0 || map_len > MOE355_MAX_EXPERTS)
    return fail(MOE355_EUNSUPPORTED, "expert_map length %d outside [0, %d]", map_len,
                MOE355_MAX_EXPERTS);
  if (map_len > 0 && !expert_map) return fail(MOE355_EINVAL, "expert_map is NULL");
  if (p->rows == 0) return MOE355_OK;
  if (!topk_ids || !workspace) return fail(MOE355_EINVAL, "NULL topk_ids or workspace");
  *a = PermuteArgs{};
  a->ids = topk_ids;
  a->block_counts = at<int32_t>(workspace, p->off_block_counts);
  a->offsets = at<int32_t>(workspace, p->off_offsets);
  a->slot_to_row = at<int32_t>(workspace, p->off_slot_to_row);
  a->row_src = at<int32_t>(workspace, p->off_row_src);
  a->tile_map = at<int32_t>(workspace, p->off_tile_map);
  a->R = p->rows; a->K = p->K; a->E = p->E; a->n_blocks = p->n_blocks;
  a->tile_rows = p->tile_rows; a->max_tiles = p->max_tiles;
  a->ids_int64 = ids_int64 != 0; a->map_len = map_len;
  for (int i = 0; i < map_len; ++i) a->map[i] = expert_map[i];
  a->weights = topk_w;
  return MOE355_OK;
}

// moe355_gate_up, or with self (skinny path, <= 64 routed slots) the
// self-permuting gate_up that also does the permute's work.
int gate_up_impl(const moe355_plan* p, const void* x, const void* const* w1, int act,
                 void* workspace, void* stream, const PermuteArgs* self);

}  // namespace

extern "C" {

// The permute; with topk_w (the fused entry points), slots of weight 0 are
// dropped as well.
int permute_impl(const moe355_plan* p, const void* topk_ids, int ids_int64,
                 const int32_t* expert_map, int map_len, const float* topk_w, void* workspace,
                 void* stream) {
  int rc = check_plan(p);
  if (rc) return rc;
  PermuteArgs a;
  if ((rc = permute_args(p, topk_ids, ids_int64, expert_map, map_len, workspace, &a, topk_w)))
    return rc;
  if (p->rows == 0) return MOE355_OK;
  return check_hip(launch_permute(a, as_stream(stream)), "permute launch");
}

int moe355_permute(const moe355_plan* p, const void* topk_ids, int ids_int64,
                   const int32_t* expert_map, int map_len, void* workspace, void* stream) {
  return permute_impl(p, topk_ids, ids_int64, expert_map, map_len, nullptr, workspace, stream);
}

int moe355_gate_up(const moe355_plan* p, const void* x, const void* const* w1, int act,
                   void* workspace, void* stream) {
  return gate_up_impl(p, x, w1, act, workspace, stream, nullptr);
}

}  // extern "C"

namespace {

int gate_up_impl(const moe355_plan* p, const void* x, const void* const* w1, int act,
                 void* workspace, void* stream, const PermuteArgs* self) {
  int rc = check_plan(p);
  if (rc) return rc;
  if (act < MOE355_ACT_SILU || act > MOE355_ACT_GELU_TANH)
    return fail(MOE355_EINVAL, "unknown activation %d", act);
  if (p->rows == 0) return MOE355_OK;
  if (!x || !workspace) return fail(MOE355_EINVAL, "NULL x or workspace");
  if (p->path != MOE355_PATH_SIMT && !aligned16(x)) return fail(MOE355_EINVAL, "x not 16-byte aligned");
  if ((rc = check_banks(p, w1, "w1"))) return rc;
  FfnArgs a{};
  a.x = x;
  a.row_src = at<int32_t>(workspace, p->off_row_src);
  a.tile_map = at<int32_t>(workspace, p->off_tile_map);
  a.offsets = at<int32_t>(workspace, p->off_offsets);
  a.out = at<void>(workspace, p->off_inter);
  a.H = p->H; a.I = p->I; a.R = p->rows; a.max_tiles = p->max_tiles;
  a.splits = 1; a.k_per_split = p->H; a.act = act;
  for (int e = 0; e < p->E; ++e) a.w[e] = w1[e];
  hipError_t err;
  if (p->path == MOE355_PATH_MFMA_TILED || p->path == MOE355_PATH_MFMA_TILED128) {
    a.n_wtiles = p->I / 128;
    a.tile_rows = p->tile_rows;
    a.ragged = ragged_tiles(p);
    // The y and part regions are free until the down projection: they hold
    // the partial tiles of the K-split tail items (256x256 fp32 each).
    a.part = at<float>(workspace, p->off_y);
    a.part_units = static_cast<int>(
        std::min<size_t>((p->workspace_bytes - p->off_y) / (256 * 256 * 4), 4096));
    err = launch_gate_up_tiled(a, p->dtype, as_stream(stream));
  } else if (p->path == MOE355_PATH_MFMA_SKINNY) {
    a.n_wtiles = p->I / 16;
    if (self) {
      a.self_permute = 1;
      a.perm = *self;
    }
    err = launch_gate_up_skinny(a, p->dtype, as_stream(stream));
  } else {
    a.n_wtiles = (p->I + 63) / 64;
    err = launch_gate_up_simt(a, p->dtype, as_stream(stream));
  }
  return check_hip(err, "gate_up launch");
}

// Whether the down projection leaves y in the layer dtype ([rows, H], one
// plane) rather than fp32 split partials: the tiled kernels with one K-split.
// This is the reference's own rounding (its `inter @ w2[e].t()` returns the
// model dtype) and halves the y traffic of down and combine. Split partials
// stay fp32 (their sum is rounded once, by the combine).
bool y_narrow(const moe355_plan* p) {
  return (p->path == MOE355_PATH_MFMA_TILED || p->path == MOE355_PATH_MFMA_TILED128) &&
         p->down_splits == 1 && p->dtype != MOE355_F32;
}

// permute -> gate_up -> down -> combine on a filled plan and a workspace of
// plan.workspace_bytes (the body of both fused_experts entry points).
int run_fused(const moe355_plan& p, const void* x, const void* const* w1, const void* const* w2,
              const float* topk_w, const void* topk_ids, int ids_int64,
              const int32_t* expert_map, int map_len, int act, void* out, int accumulate_f32,
              void* workspace, void* stream) {
  int rc;
  if (p.path == MOE355_PATH_MFMA_SKINNY && p.rows <= 64) {
    // Decode sizes (<= 64 routed slots, one wave's worth): the gate_up
    // workgroups group the routed slots themselves (one launch fewer; the
    // permute's outputs are still written for down and combine). Every
    // workgroup pays the grouping before its weight stream: a few LDS
    // operations and one wave scan, whatever the number of distinct experts
    // (an earlier form took one round per distinct expert, which made 64
    // experts top-6 at 8 tokens 132 -> 150 us, so it ran only up to 16 slots).
    PermuteArgs pa;
    if ((rc = permute_args(&p, topk_ids, ids_int64, expert_map, map_len, workspace, &pa, topk_w)))
      return rc;
    if ((rc = gate_up_impl(&p, x, w1, act, workspace, stream, &pa))) return rc;
  } else {
    if ((rc = permute_impl(&p, topk_ids, ids_int64, expert_map, map_len, topk_w, workspace,
                           stream)))
      return rc;
    if ((rc = moe355_gate_up(&p, x, w1, act, workspace, stream))) return rc;
  }
  if ((rc = moe355_down(&p, w2, workspace, stream))) return rc;
  return moe355_combine(&p, topk_w, out, accumulate_f32, workspace, stream);
}

// Device address of this device's copy of `scratch`, looked up once per
// device with that device current. The array's host-side name is only a
// handle for the runtime: kernels must be given this address.
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

int static_scratch(void* stream, void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return check_hip(e, "hipGetDevice");
  if (dev < 0 || dev >= kMaxDevices)
    return fail(MOE355_EUNSUPPORTED, "device %d outside [0, %d)", dev, kMaxDevices);
  if (stream) {
    hipDevice_t sdev = -1;
    e = hipStreamGetDevice(as_stream(stream), &sdev);
    if (e != hipSuccess) return check_hip(e, "hipStreamGetDevice");
    if (sdev != dev)
      return fail(MOE355_EINVAL, "stream is on device %d but device %d is current", sdev, dev);
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return check_hip(e, "hipGetSymbolAddress(scratch)");
    if (!p) return fail(MOE355_EHIP, "hipGetSymbolAddress(scratch) gave NULL");
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return MOE355_OK;
}

}  // namespace

extern "C" {

int moe355_down(const moe355_plan* p, const void* const* w2, void* workspace, void* stream) {
  int rc = check_plan(p);
  if (rc) return rc;
  if (p->rows == 0) return MOE355_OK;
  if (!workspace) return fail(MOE355_EINVAL, "NULL workspace");
  if ((rc = check_banks(p, w2, "w2"))) return rc;
  FfnArgs a{};
  a.x = at<void>(workspace, p->off_inter);
  a.row_src = at<int32_t>(workspace, p->off_row_src);
  a.tile_map = at<int32_t>(workspace, p->off_tile_map);
  a.offsets = at<int32_t>(workspace, p->off_offsets);
  a.out = at<void>(workspace, p->off_y);
  a.H = p->H; a.I = p->I; a.R = p->rows; a.max_tiles = p->max_tiles;
  a.splits = p->down_splits; a.k_per_split = p->I / p->down_splits; a.act = 0;
  for (int e = 0; e < p->E; ++e) a.w[e] = w2[e];
  hipError_t err;
  if (p->path == MOE355_PATH_MFMA_TILED || p->path == MOE355_PATH_MFMA_TILED128) {
    a.n_wtiles = p->H / 256;
    a.tile_rows = p->tile_rows;
    a.ragged = ragged_tiles(p);
    a.y16 = y_narrow(p);
    // Partial tiles of the K-split last-round items (256x256 fp32 each).
    a.part = at<float>(workspace, p->off_part);
    a.part_units = p->workspace_bytes > p->off_part
                       ? static_cast<int>((p->workspace_bytes - p->off_part) / (256 * 256 * 4))
                       : 0;
    err = launch_down_tiled(a, p->dtype, as_stream(stream));
  } else if (p->path == MOE355_PATH_MFMA_SKINNY) {
    a.n_wtiles = p->H / 16;
    err = launch_down_skinny(a, p->dtype, as_stream(stream));
  } else {
    a.n_wtiles = (p->H + 63) / 64;
    err = launch_down_simt(a, p->dtype, as_stream(stream));
  }
  return check_hip(err, "down launch");
}

int moe355_combine(const moe355_plan* p, const float* topk_w, void* out, int accumulate_f32,
                   void* workspace, void* stream) {
  int rc = check_plan(p);
  if (rc) return rc;
  if (p->T == 0) return MOE355_OK;
  if (!topk_w || !out || !workspace) return fail(MOE355_EINVAL, "NULL topk_w, out or workspace");
  if (!aligned16(out)) return fail(MOE355_EINVAL, "out not 16-byte aligned");
  CombineArgs a{};
  a.y = at<float>(workspace, p->off_y);
  a.topk_w = topk_w;
  a.slot_to_row = at<int32_t>(workspace, p->off_slot_to_row);
  a.out = out;
  a.T = p->T; a.K = p->K; a.H = p->H; a.R = p->rows; a.splits = p->down_splits;
  a.accumulate = accumulate_f32 != 0;
  a.y16 = y_narrow(p);
  return check_hip(launch_combine(a, p->dtype, as_stream(stream)), "combine launch");
}

int moe355_fused_experts(const void* x, const void* const* w1, const void* const* w2,
                         const float* topk_w, const void* topk_ids, int ids_int64,
                         const int32_t* expert_map, int map_len, int T, int H, int I, int E,
                         int K, int dtype, int act, void* out, int accumulate_f32,
                         void* workspace, size_t workspace_bytes, void* stream) {
  moe355_plan p;
  int rc = moe355_make_plan(T, H, I, E, K, dtype, &p);
  if (rc) return rc;
  if (T == 0) return MOE355_OK;
  if (!workspace || workspace_bytes < p.workspace_bytes)
    return fail(MOE355_EWORKSPACE, "workspace of %zu bytes, plan needs %zu", workspace_bytes,
                p.workspace_bytes);
  return run_fused(p, x, w1, w2, topk_w, topk_ids, ids_int64, expert_map, map_len, act, out,
                   accumulate_f32, workspace, stream);
}

int moe355_fused_experts_static(const void* x, const void* const* w1, const void* const* w2,
                                const float* topk_w, const void* topk_ids, int ids_int64,
                                const int32_t* expert_map, int map_len, int T, int H, int I,
                                int E, int K, int dtype, int act, void* out, int accumulate_f32,
                                void* stream) {
  moe355_plan p;
  int rc = moe355_make_plan(T, H, I, E, K, dtype, &p);
  if (rc) return rc;
  if (T == 0) return MOE355_OK;
  if (p.workspace_bytes > MOE355_STATIC_SCRATCH_BYTES) {
    // The tiled paths' last region holds one fp32 partial tile per CU for the
    // down projection's K-split tail; without it the down projection runs its
    // last round whole (same results up to fp32 summation order).
    const bool tiled = p.path == MOE355_PATH_MFMA_TILED || p.path == MOE355_PATH_MFMA_TILED128;
    if (!tiled || p.off_part > MOE355_STATIC_SCRATCH_BYTES)
      return fail(MOE355_EWORKSPACE,
                  "fused_experts_static: T=%d H=%d I=%d E=%d K=%d needs %zu bytes of scratch, "
                  "more than the library's static %u bytes; use moe355_fused_experts with a "
                  "workspace",
                  T, H, I, E, K, tiled ? p.off_part : p.workspace_bytes,
                  static_cast<unsigned>(MOE355_STATIC_SCRATCH_BYTES));
    p.workspace_bytes = p.off_part;
  }
  void* ws = nullptr;
  if ((rc = static_scratch(stream, &ws))) return rc;
  return run_fused(p, x, w1, w2, topk_w, topk_ids, ids_int64, expert_map, map_len, act, out,
                   accumulate_f32, ws, stream);
}

int moe355_cast_f32(const float* src, void* dst, size_t n, int dtype, void* stream) {
  if (!valid_dtype(dtype)) return fail(MOE355_EINVAL, "unknown dtype %d", dtype);
  if (n == 0) return MOE355_OK;
  if (!src || !dst) return fail(MOE355_EINVAL, "NULL src or dst");
  return check_hip(launch_cast_f32(src, dst, n, dtype, as_stream(stream)), "cast launch");
}

int moe355_host_staging_alloc(size_t bytes, void** host_ptr) {
  if (!host_ptr) return fail(MOE355_EINVAL, "NULL host_ptr");
  *host_ptr = nullptr;
  if (bytes == 0) return fail(MOE355_EINVAL, "zero-byte staging buffer");
  return check_hip(hipHostMalloc(host_ptr, bytes,
                                 hipHostMallocMapped | hipHostMallocCoherent |
                                     hipHostMallocPortable),
                   "hipHostMalloc (mapped, coherent)");
}

int moe355_host_staging_free(void* host_ptr) {
  if (!host_ptr) return MOE355_OK;
  return check_hip(hipHostFree(host_ptr), "hipHostFree");
}

namespace {
// The device address of a mapped pinned host pointer (interior pointers
// included); fails, and nothing is launched, for memory the runtime did not
// map for the device.
int device_view(const void* host_ptr, void** dev_ptr, const char* what) {
  *dev_ptr = nullptr;
  const hipError_t e = hipHostGetDevicePointer(dev_ptr, const_cast<void*>(host_ptr), 0);
  if (e != hipSuccess || !*dev_ptr)
    return fail(MOE355_EINVAL, "%s is not mapped pinned host memory (%s)", what,
                hipGetErrorString(e));
  return MOE355_OK;
}
}  // namespace

int moe355_copy_to_host(void* host_dst, const void* src, size_t bytes, void* stream) {
  if (bytes == 0) return MOE355_OK;
  if (!host_dst || !src) return fail(MOE355_EINVAL, "NULL host_dst or src");
  if ((reinterpret_cast<uintptr_t>(host_dst) | reinterpret_cast<uintptr_t>(src)) & 15)
    return fail(MOE355_EINVAL, "host_dst and src must be 16-byte aligned");
  void* dst = nullptr;
  if (int rc = device_view(host_dst, &dst, "host_dst")) return rc;
  return check_hip(launch_copy_bytes(src, dst, bytes, as_stream(stream)), "copy_to_host launch");
}

int moe355_copy_to_host_multi(void* host_dst, int n, const void* const* src,
                              const size_t* dst_offsets, const size_t* bytes, void* stream) {
  if (n < 0 || n > kMaxCopyRegions)
    return fail(MOE355_EINVAL, "n=%d regions outside [0, %d]", n, kMaxCopyRegions);
  if (n == 0) return MOE355_OK;
  if (!host_dst || !src || !dst_offsets || !bytes)
    return fail(MOE355_EINVAL, "NULL host_dst, src, dst_offsets or bytes");
  void* dst = nullptr;
  if (int rc = device_view(host_dst, &dst, "host_dst")) return rc;
  CopyRegions r{};
  r.count = n;
  for (int k = 0; k < n; ++k) {
    if (bytes[k] && !src[k]) return fail(MOE355_EINVAL, "NULL src[%d]", k);
    if ((reinterpret_cast<uintptr_t>(src[k]) | dst_offsets[k] |
         reinterpret_cast<uintptr_t>(host_dst)) & 15)
      return fail(MOE355_EINVAL, "src[%d], host_dst and dst_offsets[%d] must be 16-byte aligned",
                  k, k);
    r.src[k] = static_cast<const uint8_t*>(src[k]);
    r.dst[k] = static_cast<uint8_t*>(dst) + dst_offsets[k];
    r.bytes[k] = bytes[k];
  }
  return check_hip(launch_copy_regions(r, as_stream(stream)), "copy_to_host_multi launch");
}

int moe355_merge_host_f32(const float* acc, const float* host_src, size_t n, int dtype, void* out,
                          void* stream) {
  if (!valid_dtype(dtype)) return fail(MOE355_EINVAL, "unknown dtype %d", dtype);
  if (n == 0) return MOE355_OK;
  if (!acc || !host_src || !out) return fail(MOE355_EINVAL, "NULL acc, host_src or out");
  if (n % 4 || ((reinterpret_cast<uintptr_t>(acc) | reinterpret_cast<uintptr_t>(host_src)) & 15))
    return fail(MOE355_EINVAL, "n must be a multiple of 4 and acc, host_src 16-byte aligned");
  void* src = nullptr;
  if (int rc = device_view(host_src, &src, "host_src")) return rc;
  return check_hip(launch_merge_host(acc, static_cast<const float*>(src), out, n, dtype,
                                     as_stream(stream)),
                   "merge_host launch");
}

int moe355_h2d_async(void* dst, const void* src, size_t bytes, void* stream) {
  if (bytes == 0) return MOE355_OK;
  if (!dst || !src) return fail(MOE355_EINVAL, "NULL dst or src");
  return check_hip(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, as_stream(stream)),
                   "hipMemcpyAsync H2D");
}

}  // extern "C"
