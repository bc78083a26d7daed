// Wave-level softmax + top-k and a transposed wave reduction, shared by the
// router kernels (router.hip) and the fused residual add + RMSNorm + router
// kernel (norm.hip). Included inside their anonymous namespaces.
#pragma once

constexpr int kMaxPerLane = kMaxExperts / kWave;

// Softmax + top-k + renormalisation of one token's logits by one wave.
// lg: E fp32 logits (LDS or global). psel/isel: per-wave LDS scratch of E
// entries. Mirrors torch_fused_topk (fused.py:42-45) and, when kmin > 0, the
// entropy-adaptive branch of FusedMoE.route (moe_layer.py:326-342).
__device__ void wave_topk(const float* lg, int E, int K, int renorm, int kmin, float* psel,
                          int32_t* isel, float* w_out, int32_t* id_out, int lane) {
  float v[kMaxPerLane];
  bool live[kMaxPerLane];
#pragma unroll
  for (int j = 0; j < kMaxPerLane; ++j) {
    const int e = lane + kWave * j;
    live[j] = e < E;
    v[j] = live[j] ? lg[e] : -INFINITY;
  }
  float m = -INFINITY;
#pragma unroll
  for (int j = 0; j < kMaxPerLane; ++j)
    if (live[j]) m = fmaxf(m, v[j]);
  m = wave_max(m);
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < kMaxPerLane; ++j)
    if (live[j]) s += expf(v[j] - m);
  s = wave_sum(s);

  // Shannon entropy of the softmax, only for the entropy-adaptive branch.
  float hs = 0.f;
  if (kmin > 0) {
#pragma unroll
    for (int j = 0; j < kMaxPerLane; ++j) {
      if (live[j]) {
        const float p = expf(v[j] - m) / s;
        hs += p * logf(fmaxf(p, 1e-9f));
      }
    }
    hs = -wave_sum(hs);
  }

  for (int k = 0; k < K; ++k) {
    float bv = -INFINITY;
    int bi = INT_MAX;
#pragma unroll
    for (int j = 0; j < kMaxPerLane; ++j) {
      const int e = lane + kWave * j;
      if (live[j] && (v[j] > bv || (v[j] == bv && e < bi))) {
        bv = v[j];
        bi = e;
      }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      const float ov = __shfl_xor(bv, o, kWave);
      const int oi = __shfl_xor(bi, o, kWave);
      if (ov > bv || (ov == bv && oi < bi)) {
        bv = ov;
        bi = oi;
      }
    }
#pragma unroll
    for (int j = 0; j < kMaxPerLane; ++j)
      if (lane + kWave * j == bi) live[j] = false;
    if (lane == 0) {
      psel[k] = expf(bv - m) / s;
      isel[k] = bi;
    }
  }

  if (lane == 0) {
    int kd = K;
    if (kmin > 0) {
      const float hn = E > 1 ? hs / logf(static_cast<float>(E)) : 0.f;
      const float kf = rintf(static_cast<float>(kmin) + static_cast<float>(K - kmin) * hn);
      kd = static_cast<int>(fminf(fmaxf(kf, static_cast<float>(kmin)), static_cast<float>(K)));
    }
    float sum = 0.f;
    for (int k = 0; k < K; ++k) {
      const float w = k < kd ? psel[k] : 0.f;
      psel[k] = w;
      sum += w;
    }
    const bool norm = kmin > 0 || renorm;
    const float denom = kmin > 0 ? fmaxf(sum, 1e-9f) : sum;
    for (int k = 0; k < K; ++k) {
      w_out[k] = norm ? psel[k] / denom : psel[k];
      id_out[k] = isel[k];
    }
  }
}

// Wave-wide sum of V values per lane in log2(64) shuffle rounds, returning
// one total per lane: while more than one value is left, each round sends
// half of the lane's values to its partner and keeps the other half, so the V
// sums finish after 63 shuffles in total instead of 6*V. Lane l ends up with
// the sum of value index l >> (6 - log2 V).
template <int V>
__device__ __forceinline__ float transpose_reduce(float (&v)[V], int lane) {
#pragma unroll
  for (int r = 0; r < 6; ++r) {
    const int d = 32 >> r;
    const int n = (V >> r) > 1 ? (V >> r) : 1;
    if (n > 1) {
      // Bitwise select on the values: a lane-dependent `up ? v[i] : v[j]`
      // can be folded into a per-lane array index, which sends the whole
      // array to scratch memory.
      const uint32_t m = (lane & d) != 0 ? 0xffffffffu : 0u;
#pragma unroll
      for (int i = 0; i < n / 2; ++i) {
        const uint32_t lo = __float_as_uint(v[i]), hi = __float_as_uint(v[i + n / 2]);
        const float send = __uint_as_float((lo & m) | (hi & ~m));
        const float keep = __uint_as_float((hi & m) | (lo & ~m));
        v[i] = keep + __shfl_xor(send, d, kWave);
      }
    } else {
      v[0] += __shfl_xor(v[0], d, kWave);
    }
  }
  return v[0];
}

constexpr int log2i(int v) { return v <= 1 ? 0 : 1 + log2i(v / 2); }

// Softmax + top-k + renormalisation of one token by a 16-lane group (the
// lanes l .. l + 15 of one wave, sub = l % 16): lane sub holds experts
// sub + 16 j, j < NV. Selection as wave_topk (value, then lower id on exact
// ties), each reduction a 4-step butterfly inside the group. Lane sub == 0
// writes the results. K <= 8.
template <int NV>
__device__ void group16_topk(const float* lg, int E, int K, int renorm, int kmin, float* w_out,
                             int32_t* id_out, int sub) {
  float v[NV];
  bool live[NV];
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int e = sub + 16 * j;
    live[j] = e < E;
    v[j] = live[j] ? lg[e] : -INFINITY;
  }
  float m = -INFINITY;
#pragma unroll
  for (int j = 0; j < NV; ++j)
    if (live[j]) m = fmaxf(m, v[j]);
#pragma unroll
  for (int o = 8; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 16));
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < NV; ++j)
    if (live[j]) s += expf(v[j] - m);
#pragma unroll
  for (int o = 8; o > 0; o >>= 1) s += __shfl_xor(s, o, 16);
  float hs = 0.f;
  if (kmin > 0) {
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      if (live[j]) {
        const float p = expf(v[j] - m) / s;
        hs += p * logf(fmaxf(p, 1e-9f));
      }
    }
#pragma unroll
    for (int o = 8; o > 0; o >>= 1) hs += __shfl_xor(hs, o, 16);
    hs = -hs;
  }
  float psel[8];
  int isel[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    psel[k] = 0.f;
    isel[k] = 0;
    if (k >= K) continue;
    float bv = -INFINITY;
    int bi = INT_MAX;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      const int e = sub + 16 * j;
      if (live[j] && (v[j] > bv || (v[j] == bv && e < bi))) {
        bv = v[j];
        bi = e;
      }
    }
#pragma unroll
    for (int o = 8; o > 0; o >>= 1) {
      const float ov = __shfl_xor(bv, o, 16);
      const int oi = __shfl_xor(bi, o, 16);
      if (ov > bv || (ov == bv && oi < bi)) {
        bv = ov;
        bi = oi;
      }
    }
#pragma unroll
    for (int j = 0; j < NV; ++j)
      if (sub + 16 * j == bi) live[j] = false;
    psel[k] = expf(bv - m) / s;
    isel[k] = bi;
  }
  if (sub != 0) return;
  int kd = K;
  if (kmin > 0) {
    const float hn = E > 1 ? hs / logf(static_cast<float>(E)) : 0.f;
    const float kf = rintf(static_cast<float>(kmin) + static_cast<float>(K - kmin) * hn);
    kd = static_cast<int>(fminf(fmaxf(kf, static_cast<float>(kmin)), static_cast<float>(K)));
  }
  float sum = 0.f;
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    if (k < K) {
      psel[k] = k < kd ? psel[k] : 0.f;
      sum += psel[k];
    }
  }
  const bool norm = kmin > 0 || renorm;
  const float denom = kmin > 0 ? fmaxf(sum, 1e-9f) : sum;
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    if (k < K) {
      w_out[k] = norm ? psel[k] / denom : psel[k];
      id_out[k] = isel[k];
    }
  }
}
