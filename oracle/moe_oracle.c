/*
 * moe_oracle.c — CPU restatement of Reframework's MoE layer forward.
 *
 * TEST INFRASTRUCTURE ONLY. The parity tests, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library, and only as the oracle
 * the results are compared against (or the timed CPU baseline). The product (reframework_amd, libmoe355) never
 * calls it.
 *
 * Every function restates the reference algorithm in double precision, from
 * the files cited at each function (paths relative to the reference repo):
 *   oracle_router_logits  reframework/moe/moe_layer.py:323-324 (F.linear in the model dtype)
 *   oracle_topk           reframework/moe/fused.py:32-46 (+ moe_layer.py:326-342 entropy branch)
 *   oracle_permute        reframework/moe/fused.py:70-80, moe_layer.py:477-511 (remap/drop)
 *   oracle_fused_experts  reframework/moe/fused.py:49-87, reframework/layers/activation.py:15-59
 *   oracle_fused_experts_bound  the same, plus the tests' per-element bound for
 *                         fp32 evaluation (a checker bound, no reference counterpart)
 *   oracle_add_rmsnorm    reframework/layers/norm.py:27-53 (RMSNorm._forward, forward_add_residual)
 *   oracle_quantize_int8  reframework/moe/offload_cache.py:58-72 (_sym_int8_quantize)
 *   oracle_experts_int8   reframework/moe/fused.py:140-197 (fused_experts_cpu_int8), in the
 *                         reference's own fp32 / int steps rather than fp64, each slot on
 *                         its own token
 *
 * Inputs are given in their storage type (fp32, or raw bf16/f16 bits) and are
 * widened exactly. Results are fp64 (outputs) or fp32 rounded once (weights).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define ORACLE_F32 0
#define ORACLE_BF16 1
#define ORACLE_F16 2

/* ------------------------------------------------------------ conversions */
static double half_to_double(uint16_t h) {
  const int sign = (h >> 15) & 1, exp = (h >> 10) & 0x1f, man = h & 0x3ff;
  double v;
  if (exp == 0)
    v = ldexp((double)man, -24); /* subnormal: man * 2^-24 */
  else if (exp == 31)
    v = man ? NAN : INFINITY;
  else
    v = ldexp((double)(man | 0x400), exp - 25); /* (1024+man) * 2^(exp-25) */
  return sign ? -v : v;
}

static double bf16_to_double(uint16_t b) {
  uint32_t u = (uint32_t)b << 16;
  float f;
  memcpy(&f, &u, 4);
  return (double)f;
}

static double g_half_table[65536];
static int g_half_ready = 0;

static void init_half_table(void) {
  if (g_half_ready) return;
#pragma omp critical(oracle_half_table)
  {
    if (!g_half_ready) {
      for (int i = 0; i < 65536; ++i) g_half_table[i] = half_to_double((uint16_t)i);
      g_half_ready = 1;
    }
  }
}

static double load_elem(const void* base, size_t i, int type) {
  if (type == ORACLE_F32) return (double)((const float*)base)[i];
  if (type == ORACLE_BF16) return bf16_to_double(((const uint16_t*)base)[i]);
  return half_to_double(((const uint16_t*)base)[i]);
}

/* sum_i base[off + i] * v[i] over n elements of storage type `type`. */
static double dot_row(const void* base, size_t off, int type, const double* v, int n) {
  double acc = 0.0;
  if (type == ORACLE_F32) {
    const float* p = (const float*)base + off;
    for (int i = 0; i < n; ++i) acc += (double)p[i] * v[i];
  } else if (type == ORACLE_BF16) {
    const uint16_t* p = (const uint16_t*)base + off;
    for (int i = 0; i < n; ++i) acc += bf16_to_double(p[i]) * v[i];
  } else {
    const uint16_t* p = (const uint16_t*)base + off;
    for (int i = 0; i < n; ++i) acc += g_half_table[p[i]] * v[i];
  }
  return acc;
}

/* Round a double to the nearest bf16 (ties to even), returned as a double. */
static double round_bf16(double d) {
  float f = (float)d;
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7f800000u) != 0x7f800000u) {
    u += 0x7fffu + ((u >> 16) & 1u);
  }
  u &= 0xffff0000u;
  memcpy(&f, &u, 4);
  return (double)f;
}

/* Round a double to the nearest IEEE half (ties to even), returned as a double. */
static double round_f16(double d) {
  if (isnan(d) || isinf(d)) return d;
  const double a = fabs(d);
  if (a >= 65520.0) return d > 0 ? INFINITY : -INFINITY;
  int e;
  frexp(a, &e); /* a = m * 2^e, m in [0.5, 1) */
  int q = e - 11; /* spacing of halfs near a: 2^(e-11) for normals */
  if (q < -24) q = -24; /* subnormal spacing */
  const double scaled = ldexp(a, -q);
  double r = nearbyint(scaled); /* default rounding mode: ties to even */
  const double v = ldexp(r, q);
  return d < 0 ? -v : v;
}

static double round_to(double d, int mode) {
  switch (mode) {
    case 1: return round_bf16(d);
    case 2: return round_f16(d);
    case 3: return (double)(float)d;
    default: return d;
  }
}

/* -------------------------------------------------------------- activation */
static double gate_act(int act, double g) {
  if (act == 0) return g / (1.0 + exp(-g));
  if (act == 1) return 0.5 * g * (1.0 + erf(g / sqrt(2.0)));
  return 0.5 * g * (1.0 + tanh(sqrt(2.0 / M_PI) * (g + 0.044715 * g * g * g)));
}

/* ------------------------------------------------------------------ router */
/* logits[t,e] = round_model(sum_h x[t,h] gate[e,h]) + bias[e], in fp32.
 * round_mode: 0 keep fp32, 1 round to bf16, 2 round to f16 (the model dtype of
 * the reference's F.linear output). */
void oracle_router_logits(const void* x, const void* gate, int in_type, const float* bias, int T,
                          int H, int E, int round_mode, float* logits) {
#pragma omp parallel for schedule(static)
  for (int t = 0; t < T; ++t) {
    for (int e = 0; e < E; ++e) {
      double acc = 0.0;
      for (int h = 0; h < H; ++h)
        acc += load_elem(x, (size_t)t * H + h, in_type) * load_elem(gate, (size_t)e * H + h, in_type);
      float l = (float)acc;
      if (round_mode) l = (float)round_to((double)l, round_mode);
      if (bias) l = l + bias[e];
      logits[(size_t)t * E + e] = l;
    }
  }
}

/* ------------------------------------------------------------------- top-k */
/* Softmax over E (fp64), the K largest logits in descending order with exact
 * ties going to the lower expert id, weights renormalised when asked.
 * kmin > 0: entropy-adaptive k (weights past k_dyn zeroed, always renormalised
 * with a 1e-9 floor on the sum). */
int oracle_topk(const float* logits, int T, int E, int K, int renorm, int kmin, float* w_out,
                int32_t* id_out) {
  if (E < 1 || E > 256 || K < 1 || K > E) return -1;
#pragma omp parallel
  {
    char* taken = (char*)malloc((size_t)E);
    double* p = (double*)malloc(sizeof(double) * (size_t)E);
#pragma omp for schedule(static)
    for (int t = 0; t < T; ++t) {
      const float* l = logits + (size_t)t * E;
      double m = -INFINITY, s = 0.0;
      for (int e = 0; e < E; ++e) m = l[e] > m ? l[e] : m;
      for (int e = 0; e < E; ++e) {
        p[e] = exp((double)l[e] - m);
        s += p[e];
      }
      for (int e = 0; e < E; ++e) p[e] /= s;
      memset(taken, 0, (size_t)E);
      double sel[256];
      int ids[256];
      for (int k = 0; k < K; ++k) {
        int best = -1;
        for (int e = 0; e < E; ++e) {
          if (taken[e]) continue;
          if (best < 0 || l[e] > l[best]) best = e; /* strict: equal values keep the lower id */
        }
        taken[best] = 1;
        ids[k] = best;
        sel[k] = p[best];
      }
      int kd = K;
      if (kmin > 0) {
        double hs = 0.0;
        for (int e = 0; e < E; ++e) hs -= p[e] * log(p[e] > 1e-9 ? p[e] : 1e-9);
        const double hn = E > 1 ? hs / log((double)E) : 0.0;
        double kf = nearbyint((double)kmin + (double)(K - kmin) * hn);
        if (kf < kmin) kf = kmin;
        if (kf > K) kf = K;
        kd = (int)kf;
      }
      double sum = 0.0;
      for (int k = 0; k < K; ++k) {
        if (k >= kd) sel[k] = 0.0;
        sum += sel[k];
      }
      const int norm = kmin > 0 || renorm;
      const double denom = kmin > 0 ? (sum > 1e-9 ? sum : 1e-9) : sum;
      for (int k = 0; k < K; ++k) {
        w_out[(size_t)t * K + k] = (float)(norm ? sel[k] / denom : sel[k]);
        id_out[(size_t)t * K + k] = ids[k];
      }
    }
    free(taken);
    free(p);
  }
  return 0;
}

/* ----------------------------------------------------------------- permute */
/* Stable grouping of the T*K routed slots by (mapped) expert: experts
 * ascending, slots ascending within an expert. map: optional global->local
 * rename (negative = dropped); ids outside range are dropped. */
int oracle_permute(const int64_t* ids, int T, int K, int E, const int32_t* map, int map_len,
                   int32_t* offsets, int32_t* slot_to_row, int32_t* row_src) {
  const int64_t R = (int64_t)T * K;
  int32_t* local = (int32_t*)malloc(sizeof(int32_t) * (size_t)(R > 0 ? R : 1));
  int64_t* count = (int64_t*)calloc((size_t)E + 1, sizeof(int64_t));
  for (int64_t s = 0; s < R; ++s) {
    int64_t id = ids[s];
    if (map_len > 0) id = (id >= 0 && id < map_len) ? map[id] : -1;
    local[s] = (id >= 0 && id < E) ? (int32_t)id : -1;
    if (local[s] >= 0) count[local[s]]++;
  }
  int64_t acc = 0;
  for (int e = 0; e < E; ++e) {
    offsets[e] = (int32_t)acc;
    acc += count[e];
  }
  offsets[E] = (int32_t)acc;
  int64_t* next = (int64_t*)malloc(sizeof(int64_t) * (size_t)E);
  for (int e = 0; e < E; ++e) next[e] = offsets[e];
  for (int64_t r = 0; r < R; ++r) row_src[r] = -1;
  for (int64_t s = 0; s < R; ++s) {
    if (local[s] < 0) {
      slot_to_row[s] = -1;
      continue;
    }
    const int64_t row = next[local[s]]++;
    slot_to_row[s] = (int32_t)row;
    row_src[row] = (int32_t)(s / K);
  }
  free(local);
  free(count);
  free(next);
  return 0;
}

/* ----------------------------------------------------------- fused_experts */
/* out[t] = sum_k w[t,k] * down_e(act(gate_e x_t) * up_e x_t), e = ids[t,k],
 * all in fp64. w1[e] is [2I,H] (gate rows first), w2[e] is [H,I], given as
 * per-expert pointers of `w_type` elements. inter_round rounds the activated
 * intermediate to the product's storage type (0 none, 1 bf16, 2 f16, 3 f32);
 * y_round likewise rounds each slot's down-projection output y before it is
 * weighted (fused.py:83: `y = inter @ w2[e].t()` returns the model dtype).
 * Slots with id outside [0,E) contribute nothing. tokens (optional) restricts
 * the computation to the listed token indices (others left untouched). */
int oracle_fused_experts(const void* x, int x_type, const void* const* w1, const void* const* w2,
                         int w_type, const float* topk_w, const int64_t* ids, int T, int H, int I,
                         int E, int K, int act, int inter_round, int y_round,
                         const int32_t* tokens, int n_tokens, double* out) {
  const int n = tokens ? n_tokens : T;
  init_half_table();
#pragma omp parallel
  {
    double* xr = (double*)malloc(sizeof(double) * (size_t)H);
    double* inter = (double*)malloc(sizeof(double) * (size_t)I);
#pragma omp for schedule(dynamic, 1)
    for (int j = 0; j < n; ++j) {
      const int t = tokens ? tokens[j] : j;
      double* o = out + (size_t)t * H;
      for (int h = 0; h < H; ++h) {
        xr[h] = load_elem(x, (size_t)t * H + h, x_type);
        o[h] = 0.0;
      }
      for (int k = 0; k < K; ++k) {
        const int64_t e = ids[(size_t)t * K + k];
        if (e < 0 || e >= E) continue;
        const double wt = (double)topk_w[(size_t)t * K + k];
        for (int i = 0; i < I; ++i) {
          const double g = dot_row(w1[e], (size_t)i * H, w_type, xr, H);
          const double u = dot_row(w1[e], (size_t)(I + i) * H, w_type, xr, H);
          inter[i] = round_to(gate_act(act, g) * u, inter_round);
        }
        for (int h = 0; h < H; ++h)
          o[h] += wt * round_to(dot_row(w2[e], (size_t)h * I, w_type, inter, I), y_round);
      }
    }
    free(xr);
    free(inter);
  }
  return 0;
}

/* ------------------------------------------- rounding-aware checker bound */
/* Spacing of storage values (bf16: 8 significant bits; f16: 11, with the
 * subnormal spacing 2^-24 below 2^-14) around |d|, and the distance from d to
 * the nearest boundary between two neighbouring storage values. */
static double storage_spacing(double d, int mode) {
  const double a = fabs(d);
  int e = 0;
  if (a > 0.0) frexp(a, &e); /* a = m 2^e, m in [0.5, 1) */
  if (mode == 1) return ldexp(1.0, (a > 0.0 ? e : -125) - 8);
  int q = (a > 0.0 ? e : -14) - 11;
  return ldexp(1.0, q < -24 ? -24 : q);
}

static double to_boundary(double d, int mode) {
  const double s = storage_spacing(d, mode);
  const double f = fabs(d) / s;
  return fabs(f - floor(f) - 0.5) * s;
}

/* d/dg of gate_act, for the error propagation of the bound. */
static double gate_act_slope(int act, double g) {
  if (act == 0) {
    const double sg = 1.0 / (1.0 + exp(-g));
    return sg * (1.0 + g * (1.0 - sg));
  }
  if (act == 1) return 0.5 * (1.0 + erf(g / sqrt(2.0))) + g * exp(-0.5 * g * g) / sqrt(2.0 * M_PI);
  const double c = sqrt(2.0 / M_PI), z = c * (g + 0.044715 * g * g * g), t = tanh(z);
  return 0.5 * (1.0 + t) + 0.5 * g * (1.0 - t * t) * c * (1.0 + 3.0 * 0.044715 * g * g);
}

/* sum_i base[off + i] * v[i] and sum_i |base[off + i] * v[i]|. */
static double dot_row_l1(const void* base, size_t off, int type, const double* v, int n,
                         double* l1) {
  double acc = 0.0, a1 = 0.0;
  for (int i = 0; i < n; ++i) {
    const double p = load_elem(base, off + (size_t)i, type) * v[i];
    acc += p;
    a1 += fabs(p);
  }
  *l1 = a1;
  return acc;
}

/* oracle_fused_experts with inter_round / y_round given, plus, per output
 * element, how far a correct fp32 evaluation may land from it beyond the
 * output's own rounding: allow[t,h] = sum over the token's slots of |w| times
 * (a) the fp32 accumulation error of y (6 sigma of a random walk of roundings
 * of 2^-24 relative: 3 * 2^-24 * sum_i |inter_i w2_hi|), (b) for every
 * intermediate whose value v may lie on either side of a rounding boundary
 * once evaluated in fp32, the gap between its two candidate roundings times
 * |w2_hi|, and (c) the same for y itself where y is rounded. "May lie on
 * either side": the distance from v to the nearest boundary is within v's
 * fp32 error estimate, |gate_act'(g)| |u| e_g + |gate_act(g)| e_u + 2^-21 |v|
 * with e_g = 3 * 2^-24 * sum_k |x_k w1_gk| (likewise e_u), the last term for
 * the rounding of the activation (the hardware exp2 / rcp). Only bf16 and
 * f16 roundings (modes 1, 2) are bounded this way. A checker bound
 * for the tests, derived from fp32 arithmetic; not the reference's algorithm. */
int oracle_fused_experts_bound(const void* x, int x_type, const void* const* w1,
                               const void* const* w2, int w_type, const float* topk_w,
                               const int64_t* ids, int T, int H, int I, int E, int K, int act,
                               int inter_round, int y_round, const int32_t* tokens, int n_tokens,
                               double* out, double* allow) {
  const int n = tokens ? n_tokens : T;
  const double u24 = ldexp(1.0, -24);
  init_half_table();
#pragma omp parallel
  {
    double* xr = (double*)malloc(sizeof(double) * (size_t)H);
    double* inter = (double*)malloc(sizeof(double) * (size_t)I);
    double* gap = (double*)malloc(sizeof(double) * (size_t)I);
    int* flagged = (int*)malloc(sizeof(int) * (size_t)I);
#pragma omp for schedule(dynamic, 1)
    for (int j = 0; j < n; ++j) {
      const int t = tokens ? tokens[j] : j;
      double* o = out + (size_t)t * H;
      double* a = allow + (size_t)t * H;
      for (int h = 0; h < H; ++h) {
        xr[h] = load_elem(x, (size_t)t * H + h, x_type);
        o[h] = 0.0;
        a[h] = 0.0;
      }
      for (int k = 0; k < K; ++k) {
        const int64_t e = ids[(size_t)t * K + k];
        if (e < 0 || e >= E) continue;
        const double wt = (double)topk_w[(size_t)t * K + k];
        int nf = 0;
        for (int i = 0; i < I; ++i) {
          double lg, lu;
          const double g = dot_row_l1(w1[e], (size_t)i * H, w_type, xr, H, &lg);
          const double u = dot_row_l1(w1[e], (size_t)(I + i) * H, w_type, xr, H, &lu);
          const double ag = gate_act(act, g), v = ag * u;
          inter[i] = round_to(v, inter_round);
          gap[i] = 0.0;
          if (inter_round == 1 || inter_round == 2) {
            const double err = fabs(gate_act_slope(act, g) * u) * 3.0 * u24 * lg +
                               fabs(ag) * 3.0 * u24 * lu + 2.0 * u24 * 4.0 * fabs(v);
            if (to_boundary(v, inter_round) <= err) {
              gap[i] = storage_spacing(v, inter_round);
              flagged[nf++] = i;
            }
          }
        }
        for (int h = 0; h < H; ++h) {
          double ly;
          const double y = dot_row_l1(w2[e], (size_t)h * I, w_type, inter, I, &ly);
          double flip = 0.0;
          for (int f = 0; f < nf; ++f)
            flip += gap[flagged[f]] * fabs(load_elem(w2[e], (size_t)h * I + flagged[f], w_type));
          double dy = 3.0 * u24 * ly + flip;
          if ((y_round == 1 || y_round == 2) && to_boundary(y, y_round) <= dy)
            dy += storage_spacing(y, y_round);
          o[h] += wt * round_to(y, y_round);
          a[h] += fabs(wt) * dy;
        }
      }
    }
    free(xr);
    free(inter);
    free(gap);
    free(flagged);
  }
  return 0;
}

/* ---------------------------------------------------------------- rmsnorm */
/* residual_out = storage(fp32(x) + fp32(residual)) when residual != NULL (the
 * reference adds in the storage dtype: torch widens to fp32, adds, rounds
 * once), else residual_out = x; normed = storage(r * 1/sqrt(mean(r^2) + eps)
 * * w + b) with the scaling in double. w and b are doubles ([H]; b may be
 * NULL). Tensors x/residual are in storage type `type`; outputs are doubles
 * holding values representable in that type. */
void oracle_add_rmsnorm(const void* x, const void* residual, int type, const double* w,
                        const double* b, double eps, int T, int H, double* residual_out,
                        double* normed) {
  const int mode = type == ORACLE_F32 ? 3 : type;
#pragma omp parallel for schedule(static)
  for (int t = 0; t < T; ++t) {
    double* r = residual_out + (size_t)t * H;
    double ss = 0.0;
    for (int h = 0; h < H; ++h) {
      const size_t i = (size_t)t * H + h;
      double v = load_elem(x, i, type);
      if (residual) v = round_to((double)((float)v + (float)load_elem(residual, i, type)), mode);
      r[h] = v;
      ss += v * v;
    }
    const double inv = 1.0 / sqrt(ss / (double)H + eps);
    for (int h = 0; h < H; ++h)
      normed[(size_t)t * H + h] = round_to(r[h] * inv * w[h] + (b ? b[h] : 0.0), mode);
  }
}

/* Round n doubles to `mode` (1 bf16, 2 f16, 3 f32) in place; exposes the
 * rounding helpers to the Python side of the oracle. */
void oracle_round(double* v, size_t n, int mode) {
  for (size_t i = 0; i < n; ++i) v[i] = round_to(v[i], mode);
}

/* ------------------------------------------------------------------- int8 */
/* _sym_int8_quantize (reframework/moe/offload_cache.py:58-72) on n fp32
 * values: amax = max |v| (w.abs().max()); amax <= 0 -> zero codes, scale 1;
 * else scale = amax / 127.0 (an fp32 tensor divided by a Python float: fp32),
 * codes = (v / scale).round().clamp(-127, 127): fp32 true division, rounding
 * half to even. Returns the scale. */
float oracle_quantize_int8(const float* v, size_t n, int8_t* q) {
  float amax = 0.0f;
  for (size_t i = 0; i < n; ++i) {
    const float a = fabsf(v[i]);
    if (a > amax) amax = a;
  }
  if (!(amax > 0.0f)) {
    memset(q, 0, n);
    return 1.0f;
  }
  const float scale = amax / 127.0f;
  for (size_t i = 0; i < n; ++i) {
    float c = nearbyintf(v[i] / scale);
    if (c < -127.0f) c = -127.0f;
    if (c > 127.0f) c = 127.0f;
    q[i] = (int8_t)c;
  }
  return scale;
}

/* F.silu / F.gelu / F.gelu(approximate="tanh") of the gate times up, in fp32
 * as torch evaluates them elementwise (reframework/layers/activation.py:15-59):
 * silu x / (1 + exp(-x)); gelu x * 0.5 * (1 + erf(x * sqrt(1/2)));
 * tanh form 0.5 * x * (1 + tanh(sqrt(2/pi) * (x + 0.044715 * x^3))). */
static float act_mul_f32(int act, float g, float u) {
  float a;
  if (act == 0) {
    a = g / (1.0f + expf(-g));
  } else if (act == 1) {
    a = 0.5f * g * (1.0f + erff(g * 0.70710678118654752f));
  } else {
    const float c = 0.79788456080286536f;
    a = 0.5f * g * (1.0f + tanhf(c * (g + 0.044715f * g * g * g)));
  }
  return a * u;
}

/* y[t * rows + r] = sum_k a[t * n + k] * w[r * n + k], exact (int64 sums of
 * int8 products, returned as the int32 torch._int_mm gives). */
static void int_mm(const int8_t* a, int m, int n, const int8_t* w, int rows, int32_t* y) {
  for (int t = 0; t < m; ++t)
    for (int r = 0; r < rows; ++r) {
      int64_t s = 0;
      for (int k = 0; k < n; ++k) s += (int64_t)a[(size_t)t * n + k] * w[(size_t)r * n + k];
      y[(size_t)t * rows + r] = (int32_t)s;
    }
}

/* fused_experts_cpu_int8 (reframework/moe/fused.py:140-197) for n_experts
 * host experts in the order given: expert e's slots slot_offsets[e] ..
 * slot_offsets[e+1]-1, each on its own token slot_tokens[s] with weight
 * slot_weights[s]. Per expert: x rows widened to fp32 and quantized as one
 * block (xq, xs); gu = fp32(int_mm(xq, w1q)) * fp32(xs * s1) (the Python
 * float product, cast to fp32 by torch's tensor-scalar multiply);
 * inter = act(gate) * up; (iq, is) = quantize(inter block);
 * y = fp32(int_mm(iq, w2q)) * fp32(is * s2); y *= w; out[token] += y.
 * out [T, H] fp32 is accumulated. Returns 0, or -1 on bad sizes. */
int oracle_experts_int8(const void* x, int x_type, int T, int H, int I, int n_experts,
                        const int8_t* const* w1q, const int8_t* const* w2q, const float* s1,
                        const float* s2, const int32_t* slot_offsets, const int32_t* slot_tokens,
                        const float* slot_weights, int act, float* out) {
  if (T < 0 || H <= 0 || I <= 0 || n_experts < 0) return -1;
  for (int e = 0; e < n_experts; ++e) {
    const int s0 = slot_offsets[e], m = slot_offsets[e + 1] - s0;
    if (m <= 0) continue;
    float* xa = malloc(sizeof(float) * (size_t)m * H);
    int8_t* xq = malloc((size_t)m * H);
    int32_t* gu = malloc(sizeof(int32_t) * (size_t)m * 2 * I);
    float* inter = malloc(sizeof(float) * (size_t)m * I);
    int8_t* iq = malloc((size_t)m * I);
    int32_t* y = malloc(sizeof(int32_t) * (size_t)m * H);
    for (int j = 0; j < m; ++j)
      for (int h = 0; h < H; ++h)
        xa[(size_t)j * H + h] = (float)load_elem(x, (size_t)slot_tokens[s0 + j] * H + h, x_type);
    const float xs = oracle_quantize_int8(xa, (size_t)m * H, xq);
    int_mm(xq, m, H, w1q[e], 2 * I, gu);
    const float m1 = (float)((double)xs * (double)s1[e]);
    for (int j = 0; j < m; ++j)
      for (int i = 0; i < I; ++i) {
        const float g = (float)gu[(size_t)j * 2 * I + i] * m1;
        const float u = (float)gu[(size_t)j * 2 * I + I + i] * m1;
        inter[(size_t)j * I + i] = act_mul_f32(act, g, u);
      }
    const float is = oracle_quantize_int8(inter, (size_t)m * I, iq);
    int_mm(iq, m, I, w2q[e], H, y);
    const float m2 = (float)((double)is * (double)s2[e]);
    for (int j = 0; j < m; ++j) {
      float* o = out + (size_t)slot_tokens[s0 + j] * H;
      const float wt = slot_weights[s0 + j];
      for (int h = 0; h < H; ++h) {
        float v = (float)y[(size_t)j * H + h] * m2;
        v = v * wt;
        o[h] = o[h] + v;
      }
    }
    free(xa); free(xq); free(gu); free(inter); free(iq); free(y);
  }
  return 0;
}
