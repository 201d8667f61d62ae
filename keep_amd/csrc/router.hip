// Residency-biased dual top-k router: one wave64 per token.
//
// Each lane holds experts e = lane + 64*i. One evaluation of the score
// function feeds two selections: served (scores + bias_served, absent experts
// carry bias <= -1e30 and get weight 0) and demand (scores + bias_demand, the
// unmasked pool). Selection is k rounds of a wave arg-max with the total
// order "larger key, then lower index"; NaN keys rank as -inf.
#include "common.h"

namespace keep {

constexpr int RT_MAX_PER_LANE = 16;  // E <= 1024
constexpr float MASKED = -1.0e30f;

struct KeyIdx {
  float key;
  int idx;
};

__device__ __forceinline__ bool better(float ka, int ia, float kb, int ib) {
  return ka > kb || (ka == kb && ia < ib);
}

__device__ __forceinline__ KeyIdx wave_argmax(float key, int idx) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) {
    const float ok = __shfl_xor(key, m, 64);
    const int oi = __shfl_xor(idx, m, 64);
    if (better(ok, oi, key, idx)) {
      key = ok;
      idx = oi;
    }
  }
  return {key, idx};
}

// Element-wise score functions (softmax is handled with its wave reductions).
__device__ __forceinline__ float score_of(float z, int func) {
  if (func == KEEP_SCORE_SIGMOID) return 1.f / (1.f + expf(-z));
  // sqrt(softplus(z)), softplus = max(z, 0) + log1p(exp(-|z|))
  return sqrtf(fmaxf(z, 0.f) + log1pf(expf(-fabsf(z))));
}

// k rounds of selection over keys. The winners are wave-uniform; lane
// `slot0 + j` keeps winner j in a register (no dynamically indexed arrays).
template <int PER>
__device__ __forceinline__ int select_topk(const float (&key)[PER], int E, int k, int lane, int slot0) {
  uint32_t taken = 0u;
  int mine = 0;
  for (int j = 0; j < k; ++j) {
    float bk = -__builtin_inff();
    int bi = 0x7fffffff;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int e = lane + 64 * i;
      if (e < E && !((taken >> i) & 1u)) {
        float kv = key[i];
        if (kv != kv) kv = -__builtin_inff();
        if (better(kv, e, bk, bi)) {
          bk = kv;
          bi = e;
        }
      }
    }
    const KeyIdx w = wave_argmax(bk, bi);
    if (lane == slot0 + j) mine = w.idx;
    if ((w.idx & 63) == lane) taken |= 1u << (w.idx >> 6);
  }
  return mine;
}

template <int PER>
__global__ __launch_bounds__(256) void k_router(const float* logits, int T, int E, int k, const float* bias_s,
                                                const float* bias_d, int func, int renorm, float route_scale,
                                                float tau, int32_t* idx, float* w, int32_t* want, float* want_score,
                                                uint8_t* admit) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  const float* lrow = logits + (int64_t)t * E;
  float z[PER], s[PER];
  float m = -__builtin_inff();
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int e = lane + 64 * i;
    z[i] = e < E ? lrow[e] : -__builtin_inff();
    m = fmaxf(m, z[i]);
  }
  if (func == KEEP_SCORE_SOFTMAX) {
    m = wave_max(m);
    float part = 0.f;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int e = lane + 64 * i;
      s[i] = e < E ? expf(z[i] - m) : 0.f;
      part += s[i];
    }
    const float sum = wave_sum(part);
#pragma unroll
    for (int i = 0; i < PER; ++i) s[i] = s[i] / sum;
  } else {
#pragma unroll
    for (int i = 0; i < PER; ++i) s[i] = score_of(z[i], func);
  }

  float key[PER];
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int e = lane + 64 * i;
    key[i] = s[i] + (bias_s && e < E ? bias_s[e] : 0.f);
  }
  // lanes 0..k-1 receive the served winners, lanes 32..32+k-1 the demand winners
  int e_sel = select_topk<PER>(key, E, k, lane, 0);
  if (bias_d == bias_s) {
    const int same = __shfl(e_sel, lane - 32 < 0 ? 0 : lane - 32, 64);
    if (lane >= 32) e_sel = same;
  } else {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int e = lane + 64 * i;
      key[i] = s[i] + (bias_d && e < E ? bias_d[e] : 0.f);
    }
    const int d = select_topk<PER>(key, E, k, lane, 32);
    if (lane >= 32) e_sel = d;
  }

  // Lanes j < k handle served slot j, lanes 32 + j handle demand slot j. Each
  // fetches its expert's score from the owner lane (e & 63), slot e >> 6.
  const bool is_served = lane < 32;
  const int j = is_served ? lane : lane - 32;
  if (j >= k) e_sel = 0;
  float mine = 0.f;
  {
    const int owner = e_sel & 63;
    const int slot = e_sel >> 6;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const float v = __shfl(s[i], owner, 64);
      if (slot == i) mine = v;
    }
  }
  const bool valid = j < k && e_sel >= 0 && e_sel < E;
  float sv = valid ? mine : 0.f;
  bool absent = false;
  if (valid && bias_s) absent = bias_s[e_sel] <= MASKED;
  // served weights
  float wv = (is_served && valid && !absent) ? sv : 0.f;
  float wsum = 0.f;
  // deterministic sequential sum over served slots
  for (int q = 0; q < k; ++q) wsum += __shfl(wv, q, 64);
  float dv = (!is_served && valid) ? sv : 0.f;
  float dsum = 0.f;
  for (int q = 0; q < k; ++q) dsum += __shfl(dv, 32 + q, 64);
  if (valid) {
    const int64_t o = (int64_t)t * k + j;
    if (is_served) {
      idx[o] = e_sel;
      float ww = renorm ? wv / (wsum + 1e-20f) : wv;
      w[o] = ww * route_scale;
    } else {
      if (want) want[o] = e_sel;
      if (want_score) want_score[o] = sv;
      if (admit) {
        const float share = sv / (dsum + 1e-20f) * route_scale;
        admit[o] = (uint8_t)(absent && share >= tau ? 1 : 0);
      }
    }
  }
}

}  // namespace keep

using namespace keep;

extern "C" int keep_router_dual_topk(const float* logits, int64_t T, int64_t E, int64_t k, const float* bias_served,
                                     const float* bias_demand, int score_func, int renormalize, float route_scale,
                                     float tau, int32_t* idx, float* w, int32_t* want, float* want_score,
                                     uint8_t* admit, void* stream) {
  KEEP_REQUIRE(T >= 0, "T must be >= 0");
  KEEP_REQUIRE(E >= 1 && E <= 64 * RT_MAX_PER_LANE, "E must be in 1..%d, got %lld", 64 * RT_MAX_PER_LANE,
               (long long)E);
  KEEP_REQUIRE(k >= 1 && k <= 32 && k <= E, "k must be in 1..min(32, E), got %lld", (long long)k);
  KEEP_REQUIRE(score_func >= 0 && score_func <= 2, "bad score_func %d", score_func);
  if (T == 0) return KEEP_OK;
  KEEP_REQUIRE(T <= 0x7fffffffLL, "T too large");
  KEEP_REQUIRE(logits && idx && w, "logits, idx and w must be non-null");
  const unsigned blocks = (unsigned)((T + 3) / 4);
  hipStream_t s = (hipStream_t)stream;
  const int per = (int)((E + 63) / 64);
#define KEEP_ROUTER_LAUNCH(P)                                                                                   \
  hipLaunchKernelGGL((k_router<P>), dim3(blocks), dim3(256), 0, s, logits, (int)T, (int)E, (int)k, bias_served, \
                     bias_demand, score_func, renormalize, route_scale, tau, idx, w, want, want_score, admit)
  if (per <= 1) KEEP_ROUTER_LAUNCH(1);
  else if (per <= 2) KEEP_ROUTER_LAUNCH(2);
  else if (per <= 4) KEEP_ROUTER_LAUNCH(4);
  else if (per <= 6) KEEP_ROUTER_LAUNCH(6);
  else if (per <= 8) KEEP_ROUTER_LAUNCH(8);
  else KEEP_ROUTER_LAUNCH(16);
#undef KEEP_ROUTER_LAUNCH
  return launch_status("keep_router_dual_topk");
}
