// Residency-biased dual top-k for one token on one wave64 (device code shared
// by the router kernel and the fused decode-layer kernel).
//
// Lane l holds experts e = l + 64*i, i < PER. One evaluation of the score
// function feeds two selections: served (scores + bias_served; an expert with
// bias <= -1e30 is absent and gets weight 0 if picked) and demand (scores +
// bias_demand). A selection takes the k largest keys under the total order
// "larger key, then lower index", NaN keys ranking as -inf
// (scripts/v41_build/omlx_lattice.py:77-97, local_eval.py:69-91).
//
// Selection. Every (key, expert) pair becomes one 64-bit word
//   (1 << 62) | (sortable(key) << 30) | (0x3FFFFFFF - expert),
// read as a double: bit 63 is clear and the exponent field is never 0 or
// 0x7FF, so it is a positive normal number and doubles order exactly as the
// words do, i.e. as the selection order (an empty slot is +0.0, below all).
// Each lane sorts its PER words once (v_max_f64 / v_min_f64 network); a round
// is then one wave maximum of the lanes' heads (DPP inside 16-lane rows, then
// lane swaps across rows, all in vector registers), and the lane whose head
// won pops it. The winner's index is the low 30 bits of the maximum. There is
// no scalar compare or ballot chain per round.
#pragma once
#include "common.h"

namespace keep {

constexpr int RT_MAX_PER_LANE = 16;  // E <= 1024
constexpr float RT_MASKED = -1.0e30f;

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

// The float of a sortable key (rt_sortable's inverse for every non-NaN key).
__device__ __forceinline__ float rt_unsortable(uint32_t s) {
  return __uint_as_float((s & 0x80000000u) ? (s & 0x7fffffffu) : ~s);
}

// ---------------------------------------------------------------- wave reductions
//
// Inside each 16-lane row: quad_perm [1,0,3,2], quad_perm [2,3,0,1],
// row_half_mirror, row_mirror (every lane then holds its row's value). Across
// rows: row_bcast:15 into rows 1 and 3, row_bcast:31 into rows 2 and 3, so
// lane 63 holds op(op(r0, r1), op(r2, r3)), read back with one readlane.
// Disabled rows of a row_bcast step combine with 0 (the neutral element of
// every use here) and are not read.

template <int CTRL>
__device__ __forceinline__ float rt_dpp_f(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
template <int CTRL, int ROWS>
__device__ __forceinline__ float rt_bcast_f(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, ROWS, 0xF, false));
}

// Wave-uniform max / sum of v over the 64 lanes.
__device__ __forceinline__ float rt_wave_reduce(float v, bool is_max) {
#define RT_ROW(CTRL) v = is_max ? fmaxf(v, rt_dpp_f<CTRL>(v)) : v + rt_dpp_f<CTRL>(v);
#define RT_BC(CTRL, ROWS) v = is_max ? fmaxf(v, rt_bcast_f<CTRL, ROWS>(v)) : v + rt_bcast_f<CTRL, ROWS>(v);
  RT_ROW(0xB1) RT_ROW(0x4E) RT_ROW(0x141) RT_ROW(0x140)
  if (is_max) {  // max(v, 0) would be wrong for an all-negative wave: use the lane's own value instead
    v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, v),
                                                                       __builtin_bit_cast(int, v), 0x142, 0xA, 0xF,
                                                                       false)));
    v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, v),
                                                                       __builtin_bit_cast(int, v), 0x143, 0xC, 0xF,
                                                                       false)));
  } else {
    RT_BC(0x142, 0xA) RT_BC(0x143, 0xC)
  }
#undef RT_BC
#undef RT_ROW
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

// Wave-uniform max / min of unsigned 32-bit values, every lane ending with
// the result: DPP inside 16-lane rows (integer max/min take the DPP operand
// directly, with no canonicalisation of a float max), then row pairs and
// halves through v_permlane16_swap / v_permlane32_swap.
template <bool MAX>
__device__ __forceinline__ uint32_t rt_op_u32(uint32_t a, uint32_t b) {
  return MAX ? (a > b ? a : b) : (a < b ? a : b);
}
template <bool MAX, int CTRL>
__device__ __forceinline__ uint32_t rt_dpp_u32(uint32_t v) {  // folds into one v_max/min_u32_dpp
  return rt_op_u32<MAX>(v, (uint32_t)__builtin_amdgcn_mov_dpp((int)v, CTRL, 0xF, 0xF, true));
}
template <bool MAX>
__device__ __forceinline__ uint32_t rt_wave_u32(uint32_t v) {
  v = rt_dpp_u32<MAX, 0xB1>(v);   // quad_perm [1,0,3,2]
  v = rt_dpp_u32<MAX, 0x4E>(v);   // quad_perm [2,3,0,1]
  v = rt_dpp_u32<MAX, 0x141>(v);  // row_half_mirror
  v = rt_dpp_u32<MAX, 0x140>(v);  // row_mirror
  const auto p16 = __builtin_amdgcn_permlane16_swap(v, v, false, false);
  v = rt_op_u32<MAX>(p16[0], p16[1]);
  const auto p32 = __builtin_amdgcn_permlane32_swap(v, v, false, false);
  return rt_op_u32<MAX>(p32[0], p32[1]);
}
// Max over the wave of non-negative floats (or NaN, which wins), by their bits.
__device__ __forceinline__ float rt_wave_max_abs(float v) {
  return __uint_as_float(rt_wave_u32<true>(__float_as_uint(v)));
}

__device__ __forceinline__ float rt_score_of(float z, int func) {
  if (func == KEEP_SCORE_SIGMOID) return 1.f / (1.f + expf(-z));
  // sqrt(softplus(z)), softplus = max(z, 0) + log1p(exp(-|z|))
  return sqrtf(fmaxf(z, 0.f) + log1pf(expf(-fabsf(z))));
}

// ---------------------------------------------------------------- selection

__device__ __forceinline__ double rt_dkey(uint32_t sortable, int expert) {
  const uint64_t w = 0x4000000000000000ull | ((uint64_t)sortable << 30) | (uint64_t)(0x3FFFFFFFu - (uint32_t)expert);
  return sortable ? __longlong_as_double((long long)w) : 0.0;
}

template <int CTRL, int ROWS>
__device__ __forceinline__ double rt_dpp_d(double v) {
  const uint64_t u = (uint64_t)__double_as_longlong(v);
  uint32_t lo, hi;
  if constexpr (ROWS == 0xF) {
    lo = (uint32_t)__builtin_amdgcn_mov_dpp((int)(uint32_t)u, CTRL, 0xF, 0xF, false);
    hi = (uint32_t)__builtin_amdgcn_mov_dpp((int)(uint32_t)(u >> 32), CTRL, 0xF, 0xF, false);
  } else {  // disabled rows read +0.0, below every key
    lo = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)u, CTRL, ROWS, 0xF, false);
    hi = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)(u >> 32), CTRL, ROWS, 0xF, false);
  }
  return __longlong_as_double((long long)(((uint64_t)hi << 32) | lo));
}

template <bool HI>
__device__ __forceinline__ double rt_swap_max(double v) {  // max with the partner row (16) or half (32)
  const uint64_t u = (uint64_t)__double_as_longlong(v);
  const uint32_t lo = (uint32_t)u, hi = (uint32_t)(u >> 32);
  uint32_t l0, l1, h0, h1;
  if constexpr (HI) {
    const auto pl = __builtin_amdgcn_permlane32_swap(lo, lo, false, false);
    const auto ph = __builtin_amdgcn_permlane32_swap(hi, hi, false, false);
    l0 = pl[0]; l1 = pl[1]; h0 = ph[0]; h1 = ph[1];
  } else {
    const auto pl = __builtin_amdgcn_permlane16_swap(lo, lo, false, false);
    const auto ph = __builtin_amdgcn_permlane16_swap(hi, hi, false, false);
    l0 = pl[0]; l1 = pl[1]; h0 = ph[0]; h1 = ph[1];
  }
  return __builtin_fmax(__longlong_as_double((long long)(((uint64_t)h0 << 32) | l0)),
                        __longlong_as_double((long long)(((uint64_t)h1 << 32) | l1)));
}

// The largest selection word of the wave, in every lane: DPP inside 16-lane
// rows, then v_permlane16_swap (row pairs) and v_permlane32_swap (halves).
__device__ __forceinline__ uint64_t rt_wave_max_word(double v) {
  v = __builtin_fmax(v, rt_dpp_d<0xB1, 0xF>(v));
  v = __builtin_fmax(v, rt_dpp_d<0x4E, 0xF>(v));
  v = __builtin_fmax(v, rt_dpp_d<0x141, 0xF>(v));
  v = __builtin_fmax(v, rt_dpp_d<0x140, 0xF>(v));
  v = rt_swap_max<false>(v);
  v = rt_swap_max<true>(v);
  return (uint64_t)__double_as_longlong(v);
}

// The selection over the sortable keys kk (0 = no expert) of experts
// lane + 64 i, kept as state so that its rounds can run in pieces: init sorts
// each lane's words once, rounds(j0, j1, ...) finds winners j0 .. j1 - 1
// (lane slot0 + j receives winner j, or -1 when fewer than j + 1 experts hold
// a key). A block that needs only the first routes can act on them before the
// later rounds run.
template <int PER>
struct RtSel {
  uint32_t lo[PER], hi[PER];  // the sorted words as bit fields, popped with bitfield selects
  int mine;
  uint32_t mine_key;  // the sortable key of this lane's winner (0: none)

  __device__ __forceinline__ void init(const uint32_t (&kk)[PER], int lane) {
    double d[PER];
#pragma unroll
    for (int i = 0; i < PER; ++i) d[i] = rt_dkey(kk[i], lane + 64 * i);
#pragma unroll
    for (int p = 0; p < PER; ++p) {  // odd-even transposition sort, descending
#pragma unroll
      for (int i = p & 1; i + 1 < PER; i += 2) {
        const double a = d[i], b = d[i + 1];
        d[i] = __builtin_fmax(a, b);
        d[i + 1] = __builtin_fmin(a, b);
      }
    }
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const uint64_t u = (uint64_t)__double_as_longlong(d[i]);
      lo[i] = (uint32_t)u;
      hi[i] = (uint32_t)(u >> 32);
    }
    mine = -1;
    mine_key = 0u;
  }

  __device__ __forceinline__ void rounds(int j0, int j1, int lane, int slot0) {
    for (int j = j0; j < j1; ++j) {
      const uint64_t m = rt_wave_max_word(__longlong_as_double((long long)(((uint64_t)hi[0] << 32) | lo[0])));
      const uint32_t pm = (((uint64_t)hi[0] << 32) | lo[0]) == m ? 0xffffffffu : 0u;
#pragma unroll
      for (int i = 0; i + 1 < PER; ++i) {
        lo[i] = ((lo[i + 1] & pm) | (lo[i] & ~pm));
        hi[i] = (hi[i + 1] & pm) | (hi[i] & ~pm);
      }
      lo[PER - 1] &= ~pm;
      hi[PER - 1] &= ~pm;
      const int e = m ? (int)(0x3FFFFFFFu - (uint32_t)(m & 0x3FFFFFFFu)) : -1;
      mine = lane == slot0 + j ? e : mine;
      mine_key = lane == slot0 + j ? (uint32_t)(m >> 30) : mine_key;
    }
  }
};

// k rounds at once: lane slot0 + j (j < k) receives winner j, or -1; other lanes -1.
template <int PER>
__device__ __forceinline__ int rt_topk(const uint32_t (&kk)[PER], int k, int lane, int slot0) {
  RtSel<PER> sel;
  sel.init(kk, lane);
  sel.rounds(0, k, lane, slot0);
  return sel.mine;
}

struct RouteLane {
  int expert;    // the slot's expert (0 when not valid)
  float value;   // served weight (renormalised, times route_scale) / demand raw score
  uint8_t admit; // demand slots: absent and share >= tau
  bool valid;    // this lane holds a slot j < k with an expert
};

// Outputs of one selection for lane slot0 + j, j < k: the winner's score and
// served bias fetched from its owner lane, the slot sum in slot order, and
// the weight (served) or raw score and admission (demand).
template <int PER>
__device__ __forceinline__ RouteLane rt_finish(int e_sel, bool served, const float (&s)[PER],
                                               const float (&bs)[PER], int E, int k, int lane, int slot0,
                                               int renorm, float route_scale, float tau) {
  const int j = lane - slot0;
  const bool valid = j >= 0 && j < k && e_sel >= 0 && e_sel < E;
  const int e = valid ? e_sel : 0;
  const int owner = e & 63, slot = e >> 6;
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
  const float c = served ? (absent ? 0.f : sv) : sv;  // this slot's share of the sum
  float tot = 0.f;  // sequential in slot order
  for (int q = 0; q < k; ++q)
    tot += __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, c), slot0 + q));
  RouteLane r;
  r.expert = e;
  r.valid = valid;
  r.admit = 0;
  if (served) {
    r.value = (renorm ? c / (tot + 1e-20f) : c) * route_scale;
  } else {
    r.value = sv;
    r.admit = (uint8_t)(absent && sv / (tot + 1e-20f) * route_scale >= tau ? 1 : 0);
  }
  return r;
}

// Scores of the lane's experts (softmax over the wave, or the elementwise
// sigmoid / sqrt-softplus). Lanes past E hold z = -inf and score 0.
template <int PER>
__device__ __forceinline__ void rt_scores(const float (&z)[PER], int E, int func, int lane, float (&s)[PER]) {
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
    for (int i = 0; i < PER; ++i) s[i] = lane + 64 * i < E ? rt_score_of(z[i], func) : 0.f;
  }
}

template <int PER>
__device__ __forceinline__ void rt_keys(const float (&s)[PER], const float (&b)[PER], int E, int lane,
                                        uint32_t (&kk)[PER]) {
#pragma unroll
  for (int i = 0; i < PER; ++i) kk[i] = lane + 64 * i < E ? rt_sortable(s[i] + b[i]) : 0u;
}

// One token's routing on one wave: lane j < k holds served slot j, lane
// 32 + j demand slot j (k <= 32). `z` / `bs` / `bd` are the lane's logits and
// biases (experts e = lane + 64*i; lanes with e >= E hold -inf / 0).
// same_bias: the demand selection equals the served one.
template <int PER>
__device__ __forceinline__ RouteLane rt_route(const float (&z)[PER], const float (&bs)[PER], const float (&bd)[PER],
                                             int E, int k, int func, int renorm, float route_scale, float tau,
                                             bool same_bias, int lane) {
  float s[PER];
  rt_scores<PER>(z, E, func, lane, s);
  uint32_t kk[PER];
  rt_keys<PER>(s, bs, E, lane, kk);
  int e_sel = rt_topk<PER>(kk, k, lane, 0);
  if (same_bias) {
    const int same = __shfl(e_sel, lane < 32 ? 0 : lane - 32, 64);
    if (lane >= 32) e_sel = same;
  } else {
    rt_keys<PER>(s, bd, E, lane, kk);
    const int d = rt_topk<PER>(kk, k, lane, 32);
    if (lane >= 32) e_sel = d;
  }
  const RouteLane rs = rt_finish<PER>(e_sel, true, s, bs, E, k, lane, 0, renorm, route_scale, tau);
  const RouteLane rd = rt_finish<PER>(e_sel, false, s, bs, E, k, lane, 32, renorm, route_scale, tau);
  return lane < 32 ? rs : rd;
}

// The served winners alone (lane j < k: the expert of served route j, -1 for
// none; other lanes -1), equal to rt_route's served lanes. The selection
// order is "larger score + bias, then lower index"; every score function is
// increasing in the logit, so where each bias is 0 or at most RT_MASKED (no
// bias, or the residency mask) the logits order the unmasked experts as the
// keys do and the bias values order the masked ones (score + bias rounds to
// the bias there), except where score rounding makes two keys equal whose
// logits differ. For the softmax of finite logits the winners are found on
// those logit keys and certified: each winner's logit at least 2^-16 above
// the next winner's, that one within 60 of the largest logit (the difference
// z - m rounds by at most 2^-17, the exponential then differs by a factor above
// 1 + 2^-18 and the division keeps the order), or the next winner masked.
// Otherwise, or when the certificate fails, the winners come from the exact
// keys as rt_route forms them.
template <int PER>
__device__ __forceinline__ int rt_served_winners(const float (&z)[PER], const float (&bs)[PER], int E, int k,
                                                 int func, int lane) {
  bool plain = true;
#pragma unroll
  for (int i = 0; i < PER; ++i)
    plain = plain && (bs[i] == 0.f || bs[i] <= RT_MASKED) && (lane + 64 * i >= E || fabsf(z[i]) < __builtin_inff());
  if (func == KEEP_SCORE_SOFTMAX && __all(plain)) {
    uint32_t kk[PER];
#pragma unroll
    for (int i = 0; i < PER; ++i) kk[i] = lane + 64 * i < E ? rt_sortable(bs[i] != 0.f ? bs[i] : z[i]) : 0u;
    RtSel<PER> sel;
    sel.init(kk, lane);
    sel.rounds(0, min(k + 1, E), lane, 0);
    float m = -__builtin_inff();
#pragma unroll
    for (int i = 0; i < PER; ++i) m = fmaxf(m, z[i]);
    m = rt_wave_reduce(m, true);
    const uint32_t kn = (uint32_t)__shfl_down((int)sel.mine_key, 1, 64);  // winner j + 1's key (0: none)
    const float zj = rt_unsortable(sel.mine_key), zn = rt_unsortable(kn);
    const bool next_masked = kn == 0u || zn <= RT_MASKED;
    const bool ok = next_masked || (zj - zn >= 0x1p-16f && zn >= m - 60.f);
    if (__all(lane >= k || ok)) return lane < k ? sel.mine : -1;
  }
  float s[PER];
  rt_scores<PER>(z, E, func, lane, s);
  uint32_t kk[PER];
  rt_keys<PER>(s, bs, E, lane, kk);
  return rt_topk<PER>(kk, k, lane, 0);
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

// The expert -> slot map of a pool smaller than the expert count: this lane's
// entries (experts lane + 64 i), loaded beside the logits; -1 past E.
template <int PER>
__device__ __forceinline__ void rt_load_slots(const int32_t* slot_map, int E, int lane, int (&sm)[PER]) {
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int e = lane + 64 * i;
    sm[i] = e < E ? slot_map[e] : -1;
  }
}
// The slot of expert e (every lane of the wave takes part; each lane may ask
// for another expert) from its owner lane; -1 for e outside [0, E) or a slot
// outside [0, S).
template <int PER>
__device__ __forceinline__ int rt_slot_of(const int (&sm)[PER], int e, int E, int S) {
  const bool in = e >= 0 && e < E;
  const int ee = in ? e : 0;
  const int owner = ee & 63, i0 = ee >> 6;
  int v = -1;
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int x = __shfl(sm[i], owner, 64);
    v = i == i0 ? x : v;
  }
  return in && v >= 0 && v < S ? v : -1;
}

// The same routing on two waves of a block: wave 0 forms the served
// selection and wave 1 the demand selection (the served one again when the
// biases are the same), each over all experts. Scores, sums and weights are
// formed as in rt_route, so every output is bit-identical to rt_route's.
// rt_select_pair returns the slot winner of lane j < k (and the lane's scores
// for rt_finish); rt_route_pair also finishes: lane j < k of wave 0 then
// holds served slot j, of wave 1 demand slot j.
template <int PER>
__device__ __forceinline__ int rt_select_pair(const float (&z)[PER], const float (&bs)[PER], const float (&bd)[PER],
                                              int E, int k, int func, bool same_bias, int wave, int lane,
                                              float (&s)[PER]) {
  rt_scores<PER>(z, E, func, lane, s);
  uint32_t kk[PER];
  rt_keys<PER>(s, (wave == 0 || same_bias) ? bs : bd, E, lane, kk);
  return rt_topk<PER>(kk, k, lane, 0);
}

template <int PER>
__device__ __forceinline__ RouteLane rt_route_pair(const float (&z)[PER], const float (&bs)[PER],
                                                  const float (&bd)[PER], int E, int k, int func, int renorm,
                                                  float route_scale, float tau, bool same_bias, int wave,
                                                  int lane) {
  float s[PER];
  const int e_sel = rt_select_pair<PER>(z, bs, bd, E, k, func, same_bias, wave, lane, s);
  return rt_finish<PER>(e_sel, wave == 0, s, bs, E, k, lane, 0, renorm, route_scale, tau);
}

}  // namespace keep
