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
// E <= blockDim.x, k <= 8). A selection ranks instead of repeating arg-max
// rounds: every thread counts how many experts of its own wave beat it under
// the total order (a 64-bit key: the order-preserving 32-bit form of the
// score + bias above the inverted expert index, so "larger key, then lower
// index" is a plain unsigned compare). Local ranks below k are the wave's
// candidates, stored at slot wave * k + rank; one wave per selection then
// ranks the waves' candidates the same way, and rank j < k is slot j. The
// depth is 64 + nwaves * k compares, with no serial chain of reductions.
// The softmax sum is accumulated in rt_route's order (per lane over e = lane
// + 64*i, then the DPP tree), so every output is bit-identical to rt_route's.

// Block barrier for LDS traffic only (does not wait for outstanding global loads).
__device__ __forceinline__ void rt_lds_barrier() {
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0); vmcnt and expcnt left at their maxima
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// Larger key -> larger value; NaN ranks as -inf; 0 is below every key.
__device__ __forceinline__ uint32_t rt_sortable(float key) {
  if (key != key) key = -__builtin_inff();
  const uint32_t b = __float_as_uint(key + 0.0f);  // -0 -> +0
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

// Total order of the selection: larger key first, then lower expert index.
// Threads without an expert get key 0 (below every real key), still distinct.
__device__ __forceinline__ uint64_t rt_rank_key(uint32_t sortable, int expert) {
  return ((uint64_t)sortable << 32) | (uint64_t)(0xffffffffu - (uint32_t)expert);
}

struct RtCand {
  uint32_t key;  // sortable selection key (rt_sortable)
  float s, b;    // score, served bias
  int idx;       // expert
};

// LDS scratch of rt_route_block<NW, KMAX>: five disjoint 16-byte aligned arrays.
struct RtScratch {
  float* sc;       // 64 * NW + 16 floats: exp values, then the wave maxima
  uint64_t* keys;  // 64 * NW rank keys
  RtCand* cand;    // 2 * NW * KMAX candidates
  uint64_t* ckey;  // their rank keys
  RtCand* res;     // 2 * 8 winners
};
// Its size in 16-byte units, and the carving of one such buffer.
constexpr int rt_scratch_units(int nw, int kmax) {
  return (64 * nw + 16) / 4 + 64 * nw / 2 + 2 * nw * kmax + nw * kmax + 16;
}
__device__ __forceinline__ RtScratch rt_scratch(uint4* base, int nw, int kmax) {
  RtScratch m;
  m.sc = (float*)base;
  base += (64 * nw + 16) / 4;
  m.keys = (uint64_t*)base;
  base += 64 * nw / 2;
  m.cand = (RtCand*)base;
  base += 2 * nw * kmax;
  m.ckey = (uint64_t*)base;
  base += nw * kmax;
  m.res = (RtCand*)base;
  return m;
}

__device__ __forceinline__ uint64_t rt_u64_lo(uint4 v) { return ((uint64_t)v.y << 32) | v.x; }
__device__ __forceinline__ uint64_t rt_u64_hi(uint4 v) { return ((uint64_t)v.w << 32) | v.z; }

// Thread t's logit and biases (expert t), loaded unconditionally (address
// clamped, a missing bias reads the logits and is ignored) so that the number
// of loads is fixed and nothing waits for them until the routing starts.
struct RtInput {
  float z, bs, bd;
};
__device__ __forceinline__ RtInput rt_input_load(const float* lrow, const float* bias_s, const float* bias_d, int E) {
  const int t = threadIdx.x;
  const int i = t < E ? t : 0;
  return RtInput{lrow[i], (bias_s ? bias_s : lrow)[i], (bias_d ? bias_d : lrow)[i]};
}

// Rank of `mine` among 8 * NB rank keys at p, the first valid_n of them
// counted (independent counters, so the compares do not form one chain).
template <int NB>
__device__ __forceinline__ uint32_t rt_count_greater(const uint64_t* p, uint64_t mine, int valid_n) {
  uint4 q[4 * NB];
#pragma unroll
  for (int h = 0; h < 4 * NB; ++h) q[h] = *(const uint4*)(p + 2 * h);
  uint32_t c[4] = {0u, 0u, 0u, 0u};
#pragma unroll
  for (int h = 0; h < 4 * NB; ++h) {
    c[h & 3] += (2 * h < valid_n && rt_u64_lo(q[h]) > mine ? 1u : 0u) +
                (2 * h + 1 < valid_n && rt_u64_hi(q[h]) > mine ? 1u : 0u);
  }
  return (c[0] + c[1]) + (c[2] + c[3]);
}

template <int NW, int KMAX>
__device__ __forceinline__ RouteLane rt_route_block(RtInput x, bool has_bs, bool has_bd, int E, int k, int func,
                                                   int renorm, float route_scale, float tau, bool same_bias,
                                                   RtScratch m) {
  static_assert(NW % 4 == 0 && NW <= 16 && KMAX <= 8, "block router shape");
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  const int nwe = (E + 63) >> 6;  // waves that hold experts
  const bool in = t < E;
  const float z = in ? x.z : -__builtin_inff();
  const float bsw = in && has_bs ? x.bs : 0.f;
  const float bdw = in && has_bd ? x.bd : 0.f;
  float sw;
  if (func == KEEP_SCORE_SOFTMAX) {
    float* part = m.sc + 64 * NW;
    const float wm = rt_wave_reduce(z, true);
    if (lane == 0) part[w] = wm;
    rt_lds_barrier();
    float mx = -__builtin_inff();
#pragma unroll
    for (int i = 0; i < NW; i += 4) {
      const float4 q = *(const float4*)(part + i);
      mx = fmaxf(mx, fmaxf(fmaxf(q.x, q.y), fmaxf(q.z, q.w)));
    }
    const float e = in ? expf(z - mx) : 0.f;
    m.sc[t] = e;
    rt_lds_barrier();
    // every wave forms the sum itself, in rt_route's order (sc is 0 past E)
    float v[NW];
#pragma unroll
    for (int i = 0; i < NW; ++i) v[i] = m.sc[lane + 64 * i];
    float p = 0.f;
#pragma unroll
    for (int i = 0; i < NW; ++i) p += v[i];
    const float sum = rt_wave_reduce(p, false);
    sw = e / sum;
  } else {
    sw = rt_score_of(z, func);
  }
  // wave w < nwe ranks its slice, experts 64 w + lane: served (sel 0), then
  // demand (sel 1); candidates packed at sel * NW * KMAX + w * k + rank
  const int nsel = same_bias ? 1 : 2;
  if (w < nwe) {
    uint64_t* kw = m.keys + 64 * w;
    for (int sel = 0; sel < nsel; ++sel) {
      const uint32_t sk = in ? rt_sortable(sw + (sel == 0 ? bsw : bdw)) : 0u;
      const uint64_t mine = rt_rank_key(sk, t);
      kw[lane] = mine;  // read back only by this wave, after the write (in order)
      uint32_t rank = 0;
#pragma unroll
      for (int u = 0; u < 64; u += 16) rank += rt_count_greater<2>(kw + u, mine, 64 - u);
      if (rank < (uint32_t)k) {
        const int slot = sel * NW * KMAX + w * k + (int)rank;
        m.cand[slot] = RtCand{sk, sw, bsw, in ? t : 0x7fffffff};
        m.ckey[slot] = mine;
      }
      __builtin_amdgcn_wave_barrier();
    }
  }
  rt_lds_barrier();
  // merge: wave 0 served, wave 1 demand; nc = nwe * k candidates, 16 per step
  if (w < nsel) {
    const int nc = nwe * k;
    const uint64_t* ck = m.ckey + w * NW * KMAX;
    const uint64_t mine0 = lane < nc ? ck[lane] : 0u;
    const uint64_t mine1 = lane + 64 < nc ? ck[lane + 64] : 0u;
    uint32_t r0 = 0, r1 = 0;
    for (int u = 0; u < nc; u += 16) {
      r0 += rt_count_greater<2>(ck + u, mine0, nc - u);
      if (nc > 64) r1 += rt_count_greater<2>(ck + u, mine1, nc - u);
    }
    const RtCand* cw = m.cand + w * NW * KMAX;
    if (lane < nc && r0 < (uint32_t)k) m.res[w * 8 + (int)r0] = cw[lane];
    if (lane + 64 < nc && r1 < (uint32_t)k) m.res[w * 8 + (int)r1] = cw[lane + 64];
  }
  rt_lds_barrier();
  RouteLane r;
  r.valid = false;
  r.expert = 0;
  r.value = 0.f;
  r.admit = 0;
  if (w < 2 && lane < k) {
    const int src = (w == 1 && same_bias) ? 0 : w;
    RtCand o[KMAX];
#pragma unroll
    for (int q = 0; q < KMAX; ++q) o[q] = m.res[src * 8 + q];
    const RtCand c = m.res[src * 8 + lane];
    const bool valid = c.idx >= 0 && c.idx < E;
    const bool absent = valid && c.b <= RT_MASKED;
    float tot = 0.f;  // sequential over slots, as rt_route
#pragma unroll
    for (int q = 0; q < KMAX; ++q) {
      if (q < k) {
        const bool ov = o[q].idx >= 0 && o[q].idx < E;
        if (w == 0) tot += (ov && !(o[q].b <= RT_MASKED)) ? o[q].s : 0.f;
        else tot += ov ? o[q].s : 0.f;
      }
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

// ---------------------------------------------------------------- two-wave form
//
// The same routing on two waves of a block, with no LDS and no barrier: wave
// 0 forms the served selection and wave 1 the demand selection (the served
// one again when the biases are the same), each over all experts (lane l
// holds e = l + 64 i, i < PER, as rt_route). A round takes the wave maximum of
// the order-preserving 32-bit keys (rt_sortable; taken experts and lanes past
// E hold 0, below every real key), then the lowest expert index holding it
// from one ballot per slot, so a tie goes to the lower index as in rt_select;
// the winner's key is cleared. Scores, sums and weights are formed in
// rt_route's order, so every output is bit-identical to rt_route's. Result:
// lane j < k of wave 0 holds served slot j, of wave 1 demand slot j.

__device__ __forceinline__ uint32_t rt_wave_max_u32(uint32_t v) {
#define RT_MAXU(CTRL) v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xF, 0xF, false));
  RT_MAXU(0xB1) RT_MAXU(0x4E) RT_MAXU(0x141) RT_MAXU(0x140)
#undef RT_MAXU
  const uint32_t a = (uint32_t)__builtin_amdgcn_readlane((int)v, 0);
  const uint32_t b = (uint32_t)__builtin_amdgcn_readlane((int)v, 16);
  const uint32_t c = (uint32_t)__builtin_amdgcn_readlane((int)v, 32);
  const uint32_t d = (uint32_t)__builtin_amdgcn_readlane((int)v, 48);
  return max(max(a, b), max(c, d));
}

__device__ __forceinline__ float rt_readlane_f(float v, int l) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l));
}

template <int PER>
__device__ __forceinline__ RouteLane rt_route_pair(const float (&z)[PER], const float (&bs)[PER],
                                                  const float (&bd)[PER], int E, int k, int func, int renorm,
                                                  float route_scale, float tau, bool same_bias, int wave,
                                                  int lane) {
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
  const bool served = wave == 0;
  const bool use_bs = served || same_bias;
  uint32_t kk[PER];
#pragma unroll
  for (int i = 0; i < PER; ++i) kk[i] = lane + 64 * i < E ? rt_sortable(s[i] + (use_bs ? bs[i] : bd[i])) : 0u;
  RouteLane r;
  r.expert = 0;
  r.value = 0.f;
  r.admit = 0;
  r.valid = false;
  bool my_absent = false;
  float my_s = 0.f, tot = 0.f;  // tot: sequential over slots, as rt_route
  for (int j = 0; j < k; ++j) {
    uint32_t lm = kk[0];
#pragma unroll
    for (int i = 1; i < PER; ++i) lm = max(lm, kk[i]);
    const uint32_t top = rt_wave_max_u32(lm);
    int win = 0x7fffffff;
#pragma unroll
    for (int i = PER - 1; i >= 0; --i) {  // the lowest slot holding the maximum wins
      const unsigned long long b = __ballot(kk[i] == top);
      if (b != 0ull) win = 64 * i + (int)__builtin_ctzll(b);
    }
    const int wl = win & 63, wi = win >> 6;
    float sw = 0.f, bw = 0.f;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      if (i == wi) {
        sw = rt_readlane_f(s[i], wl);
        bw = rt_readlane_f(bs[i], wl);
      }
    }
#pragma unroll
    for (int i = 0; i < PER; ++i) kk[i] = (i == wi && lane == wl) ? 0u : kk[i];
    const bool valid = top != 0u && win < E;
    const bool absent = valid && bw <= RT_MASKED;
    if (!valid) sw = 0.f;
    tot += served ? ((valid && !absent) ? sw : 0.f) : sw;
    if (lane == j) {
      r.expert = valid ? win : 0;
      r.valid = valid;
      my_s = sw;
      my_absent = absent;
    }
  }
  if (served) {
    const float wv = (r.valid && !my_absent) ? my_s : 0.f;
    r.value = (renorm ? wv / (tot + 1e-20f) : wv) * route_scale;
  } else {
    r.value = my_s;
    r.admit = (uint8_t)(my_absent && my_s / (tot + 1e-20f) * route_scale >= tau ? 1 : 0);
  }
  return r;
}

}  // namespace keep
