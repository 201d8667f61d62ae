// Residency-biased dual top-k for one token on one wave64 (device code shared
// by the router kernel and the fused decode-layer kernel).
//
// Lane l holds experts e = l + 64*i, i < PER. One evaluation of the score
// function feeds two selections: served (scores + bias_served; an expert with
// bias <= -1e30 is absent and gets weight 0 if picked) and demand (scores +
// bias_demand). A selection is k rounds of a wave arg-max under the total
// order "larger key, then lower index", NaN keys ranking as -inf
// (scripts/v41_build/omlx_lattice.py:77-97, local_eval.py:69-91). Each
// round reduces inside 16-lane rows with DPP and across the four rows with
// readlane, so a round costs a few dozen cycles of latency, not a chain of
// LDS permutes.
#pragma once
#include "common.h"

namespace keep {

constexpr int RT_MAX_PER_LANE = 16;  // E <= 1024
constexpr float RT_MASKED = -1.0e30f;

__device__ __forceinline__ bool rt_better(float ka, int ia, float kb, int ib) {
  return ka > kb || (ka == kb && ia < ib);
}

__device__ __forceinline__ void rt_dpp_step(float& key, int& idx, int ctrl) {
  float ok;
  int oi;
  switch (ctrl) {  // the DPP control must be a literal
    case 0xB1:
      ok = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, key), 0xB1, 0xF, 0xF, false));
      oi = __builtin_amdgcn_update_dpp(0, idx, 0xB1, 0xF, 0xF, false);
      break;
    case 0x4E:
      ok = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, key), 0x4E, 0xF, 0xF, false));
      oi = __builtin_amdgcn_update_dpp(0, idx, 0x4E, 0xF, 0xF, false);
      break;
    case 0x141:
      ok = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, key), 0x141, 0xF, 0xF, false));
      oi = __builtin_amdgcn_update_dpp(0, idx, 0x141, 0xF, 0xF, false);
      break;
    default:
      ok = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, key), 0x140, 0xF, 0xF, false));
      oi = __builtin_amdgcn_update_dpp(0, idx, 0x140, 0xF, 0xF, false);
      break;
  }
  if (rt_better(ok, oi, key, idx)) {
    key = ok;
    idx = oi;
  }
}

// Wave-uniform arg-max of (key, idx) over 64 lanes.
__device__ __forceinline__ int rt_wave_argmax(float key, int idx) {
  rt_dpp_step(key, idx, 0xB1);   // quad_perm [1,0,3,2]
  rt_dpp_step(key, idx, 0x4E);   // quad_perm [2,3,0,1]
  rt_dpp_step(key, idx, 0x141);  // row_half_mirror
  rt_dpp_step(key, idx, 0x140);  // row_mirror: every lane of a row holds the row's best
  float bk = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, key), 0));
  int bi = __builtin_amdgcn_readlane(idx, 0);
#pragma unroll
  for (int r = 16; r < 64; r += 16) {
    const float k2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, key), r));
    const int i2 = __builtin_amdgcn_readlane(idx, r);
    if (rt_better(k2, i2, bk, bi)) {
      bk = k2;
      bi = i2;
    }
  }
  return bi;
}

// Wave-uniform max / sum: DPP inside 16-lane rows, then the four row values
// in a fixed order.
__device__ __forceinline__ float rt_row_dpp(float v, bool is_max) {
#define RT_STEP(CTRL)                                                                                               \
  {                                                                                                                 \
    const float o =                                                                                                 \
        __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false)); \
    v = is_max ? fmaxf(v, o) : v + o;                                                                               \
  }
  RT_STEP(0xB1) RT_STEP(0x4E) RT_STEP(0x141) RT_STEP(0x140)
#undef RT_STEP
  return v;
}
__device__ __forceinline__ float rt_wave_reduce(float v, bool is_max) {
  v = rt_row_dpp(v, is_max);
  const float a = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0));
  const float b = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 16));
  const float c = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 32));
  const float d = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 48));
  return is_max ? fmaxf(fmaxf(a, b), fmaxf(c, d)) : (a + b) + (c + d);
}

__device__ __forceinline__ float rt_score_of(float z, int func) {
  if (func == KEEP_SCORE_SIGMOID) return 1.f / (1.f + expf(-z));
  // sqrt(softplus(z)), softplus = max(z, 0) + log1p(exp(-|z|))
  return sqrtf(fmaxf(z, 0.f) + log1pf(expf(-fabsf(z))));
}

// k rounds of selection; returns the winners in lane order: lane slot0 + j
// holds winner j. `taken` marks the lane's own experts already selected.
template <int PER>
__device__ __forceinline__ int rt_select(const float (&key)[PER], int E, int k, int lane, int slot0) {
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
        if (rt_better(kv, e, bk, bi)) {
          bk = kv;
          bi = e;
        }
      }
    }
    const int w = rt_wave_argmax(bk, bi);
    if (lane == slot0 + j) mine = w;
    if ((w & 63) == lane) taken |= 1u << (w >> 6);
  }
  return mine;
}

struct RouteLane {
  int expert;    // lane j < k: served expert j; lane 32 + j: demanded expert j
  float value;   // served weight (renormalised, times route_scale) / demand raw score
  uint8_t admit; // demand lanes: absent and share >= tau
  bool valid;    // this lane holds slot j < k
};

// One token's routing. `z` / `bs` / `bd` are the lane's logits and biases
// (experts e = lane + 64*i; lanes with e >= E hold -inf / 0). same_bias: the
// demand selection equals the served one.
template <int PER>
__device__ __forceinline__ RouteLane rt_route(const float (&z)[PER], const float (&bs)[PER], const float (&bd)[PER],
                                             int E, int k, int func, int renorm, float route_scale, float tau,
                                             bool same_bias, int lane) {
  float s[PER];
  if (func == KEEP_SCORE_SOFTMAX) {
    float m = -__builtin_inff();
#pragma unroll
    for (int i = 0; i < PER; ++i) m = fmaxf(m, z[i]);
    m = rt_wave_reduce(m, true);
    float part = 0.f;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      s[i] = lane + 64 * i < E ? expf(z[i] - m) : 0.f;
      part += s[i];
    }
    const float sum = rt_wave_reduce(part, false);
#pragma unroll
    for (int i = 0; i < PER; ++i) s[i] = s[i] / sum;
  } else {
#pragma unroll
    for (int i = 0; i < PER; ++i) s[i] = rt_score_of(z[i], func);
  }
  float key[PER];
#pragma unroll
  for (int i = 0; i < PER; ++i) key[i] = s[i] + bs[i];
  int e_sel = rt_select<PER>(key, E, k, lane, 0);
  if (same_bias) {
    const int same = __shfl(e_sel, lane < 32 ? 0 : lane - 32, 64);
    if (lane >= 32) e_sel = same;
  } else {
#pragma unroll
    for (int i = 0; i < PER; ++i) key[i] = s[i] + bd[i];
    const int d = rt_select<PER>(key, E, k, lane, 32);
    if (lane >= 32) e_sel = d;
  }
  // Each slot lane fetches its expert's score and served bias from the owner lane.
  const bool served = lane < 32;
  const int j = served ? lane : lane - 32;
  const bool valid = j < k && e_sel >= 0 && e_sel < E;
  if (!valid) e_sel = 0;
  const int owner = e_sel & 63, slot = e_sel >> 6;
  float sv = 0.f, bv = 0.f;
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const float v = __shfl(s[i], owner, 64);
    const float b = __shfl(bs[i], owner, 64);
    if (slot == i) {
      sv = v;
      bv = b;
    }
  }
  if (!valid) sv = 0.f;
  const bool absent = valid && bv <= RT_MASKED;
  const float wv = (served && valid && !absent) ? sv : 0.f;
  const float dv = (!served && valid) ? sv : 0.f;
  float wsum = 0.f, dsum = 0.f;  // sequential sums in slot order
  for (int q = 0; q < k; ++q) {
    wsum += __shfl(wv, q, 64);
    dsum += __shfl(dv, 32 + q, 64);
  }
  RouteLane r;
  r.expert = e_sel;
  r.valid = valid;
  r.admit = 0;
  if (served) {
    r.value = (renorm ? wv / (wsum + 1e-20f) : wv) * route_scale;
  } else {
    r.value = sv;
    r.admit = (uint8_t)(absent && sv / (dsum + 1e-20f) * route_scale >= tau ? 1 : 0);
  }
  return r;
}

// Loads the lane's logits and biases (missing bias pointers read as 0).
template <int PER>
__device__ __forceinline__ void rt_load(const float* lrow, const float* bias_s, const float* bias_d, int E, int lane,
                                        float (&z)[PER], float (&bs)[PER], float (&bd)[PER]) {
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int e = lane + 64 * i;
    const bool in = e < E;
    z[i] = in ? lrow[e] : -__builtin_inff();
    bs[i] = in && bias_s ? bias_s[e] : 0.f;
    bd[i] = in && bias_d ? bias_d[e] : 0.f;
  }
}


// ---------------------------------------------------------------- block-parallel form
//
// The same routing with one thread per expert (expert t = threadIdx.x, so
// E <= blockDim.x): every wave keeps the top-k of its 64 experts, then wave 0
// merges the waves' lists for the served selection and wave 1 for the demand
// one. A selection round is a DPP max of an order-preserving 32-bit form of
// the key plus one ballot: among equal keys the lowest lane holds the lowest
// expert index, so the tie rule costs nothing in the per-wave step. The
// softmax sum is accumulated in rt_route's order (per lane over e = lane +
// 64*i, then the DPP tree), so every output is bit-identical to rt_route's.

// Block barrier for LDS traffic only (does not wait for outstanding global loads).
__device__ __forceinline__ void rt_lds_barrier() {
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0); vmcnt and expcnt left at their maxima
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// Larger key -> larger value; NaN ranks as -inf; 0 means "no candidate".
__device__ __forceinline__ uint32_t rt_sortable(float key) {
  if (key != key) key = -__builtin_inff();
  const uint32_t b = __float_as_uint(key + 0.0f);  // -0 -> +0
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

__device__ __forceinline__ uint32_t rt_wave_max_u32(uint32_t v) {
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0xB1, 0xF, 0xF, false));
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x4E, 0xF, 0xF, false));
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x141, 0xF, 0xF, false));
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x140, 0xF, 0xF, false));
  const uint32_t a = __builtin_amdgcn_readlane(v, 0), b = __builtin_amdgcn_readlane(v, 16);
  const uint32_t c = __builtin_amdgcn_readlane(v, 32), d = __builtin_amdgcn_readlane(v, 48);
  return max(max(a, b), max(c, d));
}

__device__ __forceinline__ uint32_t rt_wave_min_u32(uint32_t v) {
  v = min(v, (uint32_t)__builtin_amdgcn_update_dpp(-1, (int)v, 0xB1, 0xF, 0xF, false));
  v = min(v, (uint32_t)__builtin_amdgcn_update_dpp(-1, (int)v, 0x4E, 0xF, 0xF, false));
  v = min(v, (uint32_t)__builtin_amdgcn_update_dpp(-1, (int)v, 0x141, 0xF, 0xF, false));
  v = min(v, (uint32_t)__builtin_amdgcn_update_dpp(-1, (int)v, 0x140, 0xF, 0xF, false));
  const uint32_t a = __builtin_amdgcn_readlane(v, 0), b = __builtin_amdgcn_readlane(v, 16);
  const uint32_t c = __builtin_amdgcn_readlane(v, 32), d = __builtin_amdgcn_readlane(v, 48);
  return min(min(a, b), min(c, d));
}

struct RtCand {
  float key, s, b;  // selection key, score, served bias
  int idx;          // expert (INT_MAX: padding)
};

// Loads thread t's logit and biases unconditionally (a missing bias reads the
// logits and is ignored), so the number of loads is fixed; issue it before
// any other vector memory traffic the routing must not wait for.
struct RtInput {
  float z, bs, bd;
};
__device__ __forceinline__ RtInput rt_input_load(const float* lrow, const float* bias_s, const float* bias_d, int E) {
  const int t = threadIdx.x;
  const int i = t < E ? t : 0;
  return RtInput{lrow[i], (bias_s ? bias_s : lrow)[i], (bias_d ? bias_d : lrow)[i]};
}

// Scratch in LDS: sc[64 * nwaves + 17] floats, cand[2 * nwaves * k] records,
// res[2 * 8] records (k <= 8).
__device__ __forceinline__ RouteLane rt_route_block(RtInput x, bool has_bs, bool has_bd, int E, int k, int func,
                                                   int renorm, float route_scale, float tau, bool same_bias,
                                                   float* sc, RtCand* cand, RtCand* res) {
  const int t = threadIdx.x, lane = t & 63, w = t >> 6, nwb = blockDim.x >> 6;
  const int nwe = (E + 63) >> 6;  // waves that hold experts
  float* part = sc + 64 * nwb;
  const bool in = t < E;
  const float z = in ? x.z : -__builtin_inff();
  const float bs = in && has_bs ? x.bs : 0.f;
  const float bd = in && has_bd ? x.bd : 0.f;
  float s;
  if (func == KEEP_SCORE_SOFTMAX) {
    const float wm = rt_wave_reduce(z, true);
    if (lane == 0) part[w] = wm;
    rt_lds_barrier();
    float m = part[0];
    for (int i = 1; i < nwb; ++i) m = fmaxf(m, part[i]);
    const float e = in ? expf(z - m) : 0.f;
    sc[t] = e;
    rt_lds_barrier();
    if (w == 0) {
      float p = 0.f;
      for (int i = 0; i < nwe; ++i) p += sc[lane + 64 * i];
      const float sum = rt_wave_reduce(p, false);
      if (lane == 0) part[16] = sum;
    }
    rt_lds_barrier();
    s = e / part[16];
  } else {
    s = rt_score_of(z, func);
  }
  // per-wave top-k, served (sel 0) and demand (sel 1)
  const int nsel = same_bias ? 1 : 2;
  const RtCand pad{-__builtin_inff(), 0.f, 0.f, 0x7fffffff};
  for (int sel = 0; sel < nsel; ++sel) {
    const float key = s + (sel == 0 ? bs : bd);
    uint32_t sk = in ? rt_sortable(key) : 0u;
    for (int j = 0; j < k; ++j) {
      const uint32_t m = rt_wave_max_u32(sk);
      RtCand* dst = cand + (sel * nwb + w) * k + j;
      if (m == 0u) {
        if (lane == 0) *dst = pad;
        continue;
      }
      const uint64_t bal = __ballot(sk == m);
      if (lane == (int)__builtin_ctzll(bal)) {
        *dst = RtCand{key, s, bs, t};
        sk = 0u;
      }
    }
  }
  rt_lds_barrier();
  // merge: wave 0 served, wave 1 demand (2 candidates per lane, nwb * k <= 128)
  if (w < nsel) {
    const int nc = nwb * k;
    RtCand c0 = lane < nc ? cand[w * nc + lane] : pad;
    RtCand c1 = lane + 64 < nc ? cand[w * nc + lane + 64] : pad;
    uint32_t s0 = c0.idx != 0x7fffffff ? rt_sortable(c0.key) : 0u;
    uint32_t s1 = c1.idx != 0x7fffffff ? rt_sortable(c1.key) : 0u;
    for (int j = 0; j < k; ++j) {
      const bool first = s0 > s1 || (s0 == s1 && c0.idx < c1.idx);
      const uint32_t ls = first ? s0 : s1;
      const int li = first ? c0.idx : c1.idx;
      const uint32_t m = rt_wave_max_u32(ls);
      if (m == 0u) {
        if (lane == 0) res[w * 8 + j] = pad;
        continue;
      }
      const uint64_t bal = __ballot(ls == m);
      const uint32_t win = __builtin_popcountll(bal) == 1
                               ? (uint32_t)__builtin_amdgcn_readlane(li, (int)__builtin_ctzll(bal))
                               : rt_wave_min_u32(ls == m ? (uint32_t)li : 0xffffffffu);
      if (ls == m && (uint32_t)li == win) {
        // field-wise select: a select of whole structs goes through private memory
        res[w * 8 + j] = RtCand{first ? c0.key : c1.key, first ? c0.s : c1.s, first ? c0.b : c1.b, li};
        if (first) s0 = 0u;
        else s1 = 0u;
      }
    }
  }
  rt_lds_barrier();
  RouteLane r;
  r.valid = false;
  r.expert = 0;
  r.value = 0.f;
  r.admit = 0;
  if (w < 2 && lane < k) {
    const int src = (w == 1 && same_bias) ? 0 : w;
    const RtCand c = res[src * 8 + lane];
    const bool valid = c.idx >= 0 && c.idx < E;
    const bool absent = valid && c.b <= RT_MASKED;
    float tot = 0.f;  // sequential over slots, as rt_route
    for (int q = 0; q < k; ++q) {
      const RtCand o = res[src * 8 + q];
      const bool ov = o.idx >= 0 && o.idx < E;
      if (w == 0) tot += (ov && !(o.b <= RT_MASKED)) ? o.s : 0.f;
      else tot += ov ? o.s : 0.f;
    }
    r.valid = valid;
    r.expert = valid ? c.idx : 0;
    const float sv = valid ? c.s : 0.f;
    if (w == 0) {
      const float wv = valid && !absent ? sv : 0.f;
      r.value = (renorm ? wv / (tot + 1e-20f) : wv) * route_scale;
    } else {
      r.value = sv;
      r.admit = (uint8_t)(absent && sv / (tot + 1e-20f) * route_scale >= tau ? 1 : 0);
    }
  }
  return r;
}

}  // namespace keep
