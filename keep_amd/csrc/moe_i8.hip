// Routed MoE decode layer for one token on the int8 matrix cores of gfx950:
// router + gate/up + SwiGLU in one launch, down + combine in a second. The
// int8 decode of E8P codewords and the activation term split are described
// in q8_dev.h.
#include "common.h"
#include "moe_dev.h"
#include "q8_dev.h"
#include "route_dev.h"

namespace keep {

// T and M from the packed E8P table; flag[0] = 1 if a nibble is even (not an
// E8P half-integer coordinate, so not of this form), else 0.
__global__ __launch_bounds__(256) void k_build_tq(const uint32_t* packed, uint2* tq, uint4* tqr, uint32_t* flag) {
  __shared__ uint32_t s_bad;
  const int i = threadIdx.x;  // one block of 256 threads: abs index i, sign byte i
  if (i == 0) s_bad = 0u;
  __syncthreads();
  const uint32_t word = packed[i];
  const uint32_t p = (uint32_t)__builtin_popcount((uint32_t)i) & 1u;
  const uint32_t eff = (uint32_t)i ^ p;
  uint32_t t[2] = {0u, 0u}, m[2] = {0u, 0u};
  bool ok = true;
#pragma unroll
  for (int s = 0; s < 8; ++s) {
    const int v = (int)((word >> (4 * s)) & 15u) - 8;
    ok = ok && (v & 1) != 0;
    const int av = (v - 1) >> 1;  // v = 2a + 1
    const uint32_t tb = ((uint32_t)(av * 4 + 3)) & 0xffu;
    const uint32_t mb = (((eff >> s) & 1u) ? 0xFCu : 0u) ^ (p ? 0x02u : 0u);
    t[s >> 2] |= tb << (8 * (s & 3));
    m[s >> 2] |= mb << (8 * (s & 3));
  }
  tq[i] = make_uint2(t[0], t[1]);
  tq[256 + i] = make_uint2(m[0], m[1]);
#pragma unroll
  for (int r = 0; r < 16; ++r) tqr[i * 16 + r] = make_uint4(t[0], t[1], m[0], m[1]);
  if (!ok) s_bad = 1u;
  __syncthreads();
  if (i == 0) flag[0] = s_bad;
}

// The nested 3-bit tier: experts with a residual row (hot[e] in [0, nhot);
// -1 = none, anything else is invalid and gives NaN) add an 8-bit E8
// residual projection (codes uint8 [nhot, N, K/8], scales [nhot, N, G]) to
// the E8P base. A cold tile's residual codes come from a buffer load with no
// records, which returns zeros without touching memory, so every tile issues
// the same loads and the wait counts stay exact.
struct MQNest {
  const int32_t* hot;  // [E]
  int32_t nhot;
  const uint8_t *gc, *uc, *dc;
  const void *gs, *us, *ds;
  int sdt;
  int32_t Gh, gsz_h, Gi, gsz_i;
  const uint4* t8;    // T8R_BYTES residual image (keep_e8_1bit_image)
  int32_t* hot_route;  // [k] the routes' residual rows, written by the gate/up launch for the down launch
};

__device__ __forceinline__ uint2 res_load8(const uint8_t* row0, uint32_t bytes, uint32_t off) {
  const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc((void*)row0, (short)0, (int)bytes, 0x00020000);
  const auto v = __builtin_amdgcn_raw_buffer_load_b64(r, (int)off, 0, 0);
  return make_uint2(v[0], v[1]);
}

// Residual B operands of 8 codewords (one code byte each) -> the layout of q8_decode8.
__device__ __forceinline__ void t8_decode8(const char* img, uint32_t lane, uint2 w, q8v4 B[4]) {
  B[0] = t8_decode2(img, lane, w.x);
  B[1] = t8_decode2(img, lane, w.x >> 16);
  B[2] = t8_decode2(img, lane, w.y);
  B[3] = t8_decode2(img, lane, w.y >> 16);
}

// ------------------------------------------------------------------ router + gate/up

// The rest of the gate/up launch's arguments (the ones read first, before
// any other, are kernel arguments of their own: see k_moeq_route_gateup).
struct MQLayer {
  int func, renorm, same_bias;
  float route_scale, tau;
  int32_t k;
  const int32_t* slot_map;  // expert -> pool row (null: the pool holds every expert)
  int32_t S;                // pool rows
  int32_t* idx_out;
  float* w_out;
  int32_t* want_out;
  float* want_score_out;
  uint8_t* admit_out;
  int32_t H, I;
  const uint16_t *gc, *uc;
  const void *gs, *us;
  int sdt;
  int32_t Gh, gsz_h;
  const uint32_t* tq_bad;
  float limit;
  uint16_t* h;  // [k, I] bf16
  int32_t qtiles;
  MQNest n;  // RES only
};

// One block per NT / 2 q-tiles (16 rows of the [k, I] intermediate each), 16
// waves, H = 4096 (a 256-wide K slice per wave). Wave 0 selects the routes the
// block's own tiles belong to while waves 2-15 build the A terms of all
// sixteen slices; after one barrier every wave issues all of its scale and
// code loads at once, block 0's waves 0 and 1 finish the served and demand
// selections and write the router's outputs while those are in flight, and
// gate/up runs tile by tile, then SwiGLU, h in bf16. The arguments the first
// loads need (logits, biases, the table image, x and E) come first and are
// preloaded into SGPRs by the dispatcher (-amdgpu-kernarg-preload-count), so
// no load waits for a kernel-argument fetch. RES: the nested tier's
// residual image and hot[] come into LDS with the table, and a tile of a hot
// expert adds its residual dot (same A terms) before the SwiGLU.
template <int NT, bool XBF, int PER, bool RES>
__global__ __launch_bounds__(1024) void k_moeq_route_gateup(const float* logits, const float* bias_s,
                                                            const float* bias_d, const uint4* tqr, const void* xin,
                                                            int32_t E, MQLayer a) {
  __shared__ uint4 tqs[TQR_BYTES / 16];
  __shared__ uint4 t8s[RES ? T8R_BYTES / 16 : 1];
  __shared__ int32_t s_hot[RES ? 1024 : 1];
  __shared__ uint4 ash[16 * 3 * 16];  // [slice][term][g * 4 + i]
  __shared__ float gred[16 * NT * 16];
  __shared__ float s_inv4s[16];
  __shared__ int32_t s_idx[8];
  constexpr int QT = NT / 2;
  const char* tq = (const char*)tqs;
  const Q8Keys lk = q8_keys(threadIdx.x & 63);
  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t j = lane & 15, g = lane >> 4;
  const uint32_t C = (uint32_t)a.H >> 3;  // 512 token chunks

  // 0. the router's inputs (waves 0, 1), the table image (64 KiB; every wave
  //    DMAs 4 KiB) and the token slices this wave builds A terms for (16
  //    bytes per lane pair): wave w >= 2 slice w, waves 2 and 3 also slices 0,
  //    1. These use the preloaded arguments only; what needs the others (the
  //    table flag, the slot map, the nested tier) is issued after them.
  const uint32_t b = blockIdx.x;
  float z[PER], bsv[PER], bdv[PER];
  int sm[PER];
  if (wv == 0 || (wv == 1 && b == 0)) rt_load<PER>(logits, bias_s, bias_d, E, lane, z, bsv, bdv);
#pragma unroll
  for (int u = 0; u < 4; ++u) dma16_q(tqr + (wv * 4 + u) * 64 + lane, tqs + (wv * 4 + u) * 64);
  const uint4 xc = ldg16_q((const uint4*)xin + (wv < 2 ? 0 : wv) * 32 + (lane >> 1));
  const uint4 xc2 = ldg16_q((const uint4*)xin + (wv < 4 ? (wv & 1) : 0) * 32 + (lane >> 1));
  __builtin_amdgcn_sched_barrier(0);
  const uint32_t tq_bad = ((const __attribute__((address_space(4))) uint32_t*)a.tq_bad)[0];
  if (wv == 0 && a.slot_map) rt_load_slots<PER>(a.slot_map, E, lane, sm);
  if constexpr (RES) {
#pragma unroll
    for (int u = 0; u < 2; ++u) dma16_q(a.n.t8 + (wv * 2 + u) * 64 + lane, t8s + (wv * 2 + u) * 64);
    if (wv >= 2) {  // hot[0 .. E): 64 entries per wave, waves 2 and 3 also 896 ..
      const int i0 = (wv - 2) * 64;
      dma4_q(a.n.hot + min(i0 + lane, a.S - 1), (uint32_t*)s_hot + i0);
      if (wv < 4 && a.S > 896) dma4_q(a.n.hot + min(896 + i0 + lane, a.S - 1), (uint32_t*)s_hot + 896 + i0);
    }
  }
  __builtin_amdgcn_sched_barrier(0);

  // 1. the block's routes (wave 0) | A terms: rows 0-2 of slice w are the
  //    three int8 terms of x s, s the slice's power of two (1 / (4 s) kept for
  //    the epilogue). The block's tiles lie in routes 0 .. kneed - 1; the later
  //    selection rounds run only in block 0, once its codes are in flight.
  float sc[PER];
  int e_sel = -1, sl = -1;
  const int qlast = min((int)(b * QT + QT - 1), a.qtiles - 1);
  const int kneed = qlast < (int)(b * QT) ? 1 : min(a.k, qlast * 16 / a.I + 1);
  RtSel<PER> sel;
  auto build = [&](uint4 c, int slice) {
    float v[4];
    q8_half4<XBF>(c, lane & 1, v);
    float mx = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
    float s, inv4s;
    q8_scale(rt_wave_reduce(mx, true), s, inv4s);
    uint32_t tw[3];
    q8_terms<3>(v, s, tw);
    uint32_t* aw = (uint32_t*)ash;
#pragma unroll
    for (int n = 0; n < 3; ++n) aw[q8_aword((uint32_t)(slice * 3 + n), lane >> 1, lane & 1)] = tw[n];
    if (lane == 0) s_inv4s[slice] = inv4s;
  };
  if (wv == 0) {
    rt_scores<PER>(z, E, a.func, lane, sc);
    uint32_t kk[PER];
    rt_keys<PER>(sc, bsv, E, lane, kk);
    sel.init(kk, lane);
    sel.rounds(0, kneed, lane, 0);
    e_sel = sel.mine;
    sl = a.slot_map ? rt_slot_of<PER>(sm, e_sel, E, a.S) : (e_sel >= 0 && e_sel < E ? e_sel : -1);
    if (lane < kneed) s_idx[lane] = sl;
  } else if (wv >= 2) {
    build(xc, wv);
    if (wv < 4) build(xc2, wv - 2);
  }
  wait_vm_q<0>();  // this wave's table pieces
  rt_lds_barrier();  // the block's routes in s_idx, the table and every slice's A terms visible

  // 2. this block's tiles: scales, then every tile's codes
  uint32_t rbase[QT], rres[QT];
  bool hot_t[QT];
#pragma unroll
  for (int u = 0; u < QT; ++u) {
    const uint32_t qt = b * QT + u;
    const bool valid = qt < (uint32_t)a.qtiles;
    const uint32_t q0 = (valid ? qt : 0u) * 16u;
    const uint32_t route = q0 / (uint32_t)a.I;
    const int32_t e = s_idx[route];
    const bool ok = valid && e >= 0 && e < a.S;
    rbase[u] = (ok ? (uint32_t)e * (uint32_t)a.I : 0u) + (q0 - route * (uint32_t)a.I);
    if constexpr (RES) {
      const int32_t hr = __builtin_amdgcn_readfirstlane(ok ? s_hot[e] : -1);
      hot_t[u] = hr >= 0 && hr < a.n.nhot;
      rres[u] = (hot_t[u] ? (uint32_t)hr * (uint32_t)a.I : 0u) + (q0 - route * (uint32_t)a.I);
    }
  }
  const uint32_t grp = (uint32_t)(wv * 256) / (uint32_t)a.gsz_h;
  // per-row gate and up scales (g1): a tile's slice partials are summed unscaled and the row scale
  // applied once to the sum (a hot tile of the tier excepted: its residual has scales of its own), so
  // only the reducing lanes (wave 0, lane 16 u + jj: row jj of q-tile u) load scale words
  const bool g1 = a.gsz_h == 4096;
  ScaleRaw sr[NT], srow[2] = {0u, 0u};
#pragma unroll
  for (int t = 0; t < NT; ++t) sr[t] = 0u;
  if (!g1 || RES) {
#pragma unroll
    for (int u = 0; u < QT; ++u) {
      const uint32_t si = (rbase[u] + j) * (uint32_t)a.Gh + grp;
      sr[2 * u] = scale_raw(a.gs, a.sdt, si);
      sr[2 * u + 1] = scale_raw(a.us, a.sdt, si);
    }
  }
  if (g1) {
    uint32_t rb = rbase[0];
#pragma unroll
    for (int u = 1; u < QT; ++u) rb = (lane >> 4) == (uint32_t)u ? rbase[u] : rb;
    const bool ld = wv == 0 && lane < QT * 16;
    srow[0] = ld ? scale_raw(a.gs, a.sdt, rb + j) : 0u;
    srow[1] = ld ? scale_raw(a.us, a.sdt, rb + j) : 0u;
  }
  constexpr int PD = NT;  // tiles whose codes are loaded before the first decode
  const uint32_t kc0 = wv * 32 + g * 8;
  uint4 q[NT];
  auto load_tile = [&](int t) { q[t] = ldg16_q(((t & 1) ? a.uc : a.gc) + (size_t)(rbase[t >> 1] + j) * C + kc0); };
#pragma unroll
  for (int t = 0; t < PD; ++t) load_tile(t);
  // residual scales and codes (C bytes per row: one byte per codeword)
  const uint32_t rgrp = RES ? (uint32_t)(wv * 256) / (uint32_t)a.n.gsz_h : 0u;
  ScaleRaw srr[NT];
  uint2 qr[NT];
  if constexpr (RES) {
#pragma unroll
    for (int u = 0; u < QT; ++u) {
      const uint32_t si = (rres[u] + j) * (uint32_t)a.n.Gh + rgrp;
      srr[2 * u] = scale_raw(a.n.gs, a.n.sdt, si);
      srr[2 * u + 1] = scale_raw(a.n.us, a.n.sdt, si);
    }
#pragma unroll
    for (int t = 0; t < NT; ++t)
      qr[t] = res_load8(((t & 1) ? a.n.uc : a.n.gc) + (size_t)rres[t >> 1] * C, hot_t[t >> 1] ? 16u * C : 0u,
                        j * C + kc0);
  }
  __builtin_amdgcn_sched_barrier(0);

  // block 0: the remaining served routes (wave 0) and the demand selection
  // (wave 1), their weights and the router's outputs, while the codes are in
  // flight (s_idx of the later routes is read only after the next barrier)
  if (b == 0 && wv < 2) {
    if (wv == 0) {
      sel.rounds(kneed, a.k, lane, 0);
      e_sel = sel.mine;
      sl = a.slot_map ? rt_slot_of<PER>(sm, e_sel, E, a.S) : (e_sel >= 0 && e_sel < E ? e_sel : -1);
      if (lane >= kneed && lane < a.k) s_idx[lane] = sl;
    } else {
      e_sel = rt_select_pair<PER>(z, bsv, bdv, E, a.k, a.func, a.same_bias != 0, 1, lane, sc);
    }
    const RouteLane r = rt_finish<PER>(e_sel, wv == 0, sc, bsv, E, a.k, lane, 0, a.renorm, a.route_scale, a.tau);
    if (r.valid) {
      if (wv == 0) {
        a.idx_out[lane] = sl;  // the pool row (the expert itself without a slot map)
        a.w_out[lane] = r.value;
      } else {
        if (a.want_out) a.want_out[lane] = r.expert;
        if (a.want_score_out) a.want_score_out[lane] = r.value;
        if (a.admit_out) a.admit_out[lane] = r.admit;
      }
    }
  }

  q8v4 A[4];
  {
    const q8v4* as = (const q8v4*)ash + (wv * 3 + (j < 3 ? j : 0)) * 16 + g * 4;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const q8v4 v = as[i];
      A[i] = j < 3 ? v : q8v4{0, 0, 0, 0};
    }
  }
  const float inv4s = s_inv4s[wv];

  // 3. gate/up, tile by tile
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    if (t + PD < NT) load_tile(t + PD);
    __builtin_amdgcn_sched_barrier(0);
    q8v4 B[4];
    q8_decode8(tq, lk, q[t], B);
    q8v4 acc = {0, 0, 0, 0};
#pragma unroll
    for (int i = 0; i < 4; ++i) acc = mfma_i8(A[i], B[i], acc);
    float vr = 0.f;
    if constexpr (RES) {
      if (hot_t[t >> 1]) {  // block-uniform
        q8v4 R[4];
        t8_decode8((const char*)t8s, (uint32_t)lane, qr[t], R);
        q8v4 accr = {0, 0, 0, 0};
#pragma unroll
        for (int i = 0; i < 4; ++i) accr = mfma_i8(A[i], R[i], accr);
        const float dr = ((float)accr[0] + (float)accr[1] * 0.0078125f) + (float)accr[2] * 0.00006103515625f;
        vr = dr * inv4s * scale_cvt(srr[t], a.n.sdt, (rres[t >> 1] + j) * (uint32_t)a.n.Gh + rgrp);
      }
    }
    const uint32_t si = (rbase[t >> 1] + j) * (uint32_t)a.Gh + grp;
    const bool fold = g1 && !(RES && hot_t[t >> 1]);  // block-uniform
    if (lane < 16) {
      const float d = ((float)acc[0] + (float)acc[1] * 0.0078125f) + (float)acc[2] * 0.00006103515625f;
      gred[(wv * NT + t) * 16 + j] = fold ? d * inv4s : d * inv4s * scale_cvt(sr[t], a.sdt, si) + vr;
    }
  }
  rt_lds_barrier();
  if (wv == 0 && lane < QT * 16) {
    const uint32_t u = lane >> 4, jj = lane & 15;
    const uint32_t qt = blockIdx.x * QT + u;
    float gsum = 0.f, usum = 0.f;
    for (int w = 0; w < 16; ++w) {
      gsum += gred[(w * NT + 2 * u) * 16 + jj];
      usum += gred[(w * NT + 2 * u + 1) * 16 + jj];
    }
    bool hot_u = false;
    if constexpr (RES) {
#pragma unroll
      for (int v = 0; v < QT; ++v) hot_u = u == (uint32_t)v ? hot_t[v] : hot_u;
    }
    if (g1 && !hot_u) {
      uint32_t rb = rbase[0];
#pragma unroll
      for (int v = 1; v < QT; ++v) rb = u == (uint32_t)v ? rbase[v] : rb;
      gsum *= scale_cvt(srow[0], a.sdt, rb + jj);
      usum *= scale_cvt(srow[1], a.sdt, rb + jj);
    }
    if (qt < (uint32_t)a.qtiles) {
      const uint32_t q0 = qt * 16u;
      const int32_t e = s_idx[q0 / (uint32_t)a.I];
      float hv = silu_mul(gsum, usum, a.limit);
      if (tq_bad) hv = __builtin_nanf("");
      if constexpr (RES) {
        const int32_t hr = e >= 0 && e < a.S ? s_hot[e] : -1;
        if (hr < -1 || hr >= a.n.nhot) hv = __builtin_nanf("");
      }
      if (e >= 0 && e < a.S) a.h[q0 + jj] = from_float<bf16s>(hv).bits;
    }
  }
  if constexpr (RES) {
    if (blockIdx.x == 0 && wv == 0 && lane < a.k) {
      const int32_t e = s_idx[lane];
      a.n.hot_route[lane] = e >= 0 && e < a.S ? s_hot[e] : -1;
    }
  }
}

// ------------------------------------------------------------------ down + combine

// The rest of the down launch's arguments (see k_moeq_down for the first ones).
struct MQDown {
  int32_t H, E;
  const uint16_t* dc;
  const void* ds;
  int sdt;
  int32_t Gi, gsz_i;
  const uint32_t* tq_bad;
  void* out;
  int odt;
  MQNest n;  // RES only
};

// One block per 16 output rows, 8 waves (I / 256 of them decode a 256-wide K
// slice). A rows 2r and 2r + 1 hold the two int8 terms of route r's h slice
// (x its own scale); route r's dot is D rows 2r, 2r + 1. RES: a route with a
// residual row (hot_route, from the gate/up launch) adds its residual dot.
// The routes, the table image, h and I are the first (SGPR-preloaded) arguments.
template <int KMAX, bool RES>
__global__ __launch_bounds__(512) void k_moeq_down(const int32_t* idx, const float* wts, const uint4* tqr,
                                                   const uint16_t* hin, int32_t I, MQDown a) {
  static_assert(KMAX <= 8, "two A rows per route");
  __shared__ uint4 tqs[TQR_BYTES / 16];
  __shared__ uint4 t8s[RES ? T8R_BYTES / 16 : 1];
  __shared__ uint4 ash[8 * 2 * KMAX * 16];  // [wave][2 r + term][g * 4 + i]
  __shared__ float red[8][KMAX][16];
  const char* tq = (const char*)tqs;
  const Q8Keys lk = q8_keys(threadIdx.x & 63);
  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nwd = I >> 8;
  const bool dec = wv < nwd;  // wave-uniform
  const uint32_t j = lane & 15, g = lane >> 4;
  const uint32_t C = (uint32_t)I >> 3;
  const uint32_t n0 = blockIdx.x * 16;

  // 1. routes (scalar loads; KMAX == k), the table (8 pieces), this wave's h
  //    slices, all from preloaded arguments; then what needs the others
  typedef const __attribute__((address_space(4))) int32_t* cidx;
  typedef const __attribute__((address_space(4))) float* cw;
  int32_t e_r[KMAX], h_r[KMAX];
  float w_r[KMAX];
#pragma unroll
  for (int r = 0; r < KMAX; ++r) {
    e_r[r] = ((cidx)idx)[r];
    w_r[r] = ((cw)wts)[r];
  }
#pragma unroll
  for (int u = 0; u < 8; ++u) dma16_q(tqr + (wv * 8 + u) * 64 + lane, tqs + (wv * 8 + u) * 64);
  const uint32_t wslice = (dec ? wv : 0) * 32 + (lane >> 1);
  uint4 hq[KMAX];
#pragma unroll
  for (int r = 0; r < KMAX; ++r) hq[r] = ldg16_q((const uint4*)(hin + (size_t)r * I) + wslice);
  __builtin_amdgcn_sched_barrier(0);
  const uint32_t tq_bad = ((const __attribute__((address_space(4))) uint32_t*)a.tq_bad)[0];
  if constexpr (RES) {
#pragma unroll
    for (int r = 0; r < KMAX; ++r) h_r[r] = ((cidx)a.n.hot_route)[r];
#pragma unroll
    for (int u = 0; u < 4; ++u) dma16_q(a.n.t8 + (wv * 4 + u) * 64 + lane, t8s + (wv * 4 + u) * 64);
  }
  __builtin_amdgcn_sched_barrier(0);
  uint32_t dbase[KMAX], rres[KMAX];
  bool hot[KMAX];
  float wt[KMAX];
  bool bad = false;
#pragma unroll
  for (int r = 0; r < KMAX; ++r) {
    const bool ok = e_r[r] >= 0 && e_r[r] < a.E;
    bad |= w_r[r] != 0.f && !ok;
    wt[r] = ok ? w_r[r] : 0.f;
    dbase[r] = (ok ? (uint32_t)e_r[r] * (uint32_t)a.H : 0u) + n0;
    if constexpr (RES) {
      hot[r] = ok && h_r[r] >= 0 && h_r[r] < a.n.nhot;
      bad |= w_r[r] != 0.f && ok && (h_r[r] < -1 || h_r[r] >= a.n.nhot);
      rres[r] = (hot[r] ? (uint32_t)h_r[r] * (uint32_t)a.H : 0u) + n0;
    }
  }

  // 2. scales and codes (route r loaded PD routes ahead of its decode; RES: every residual up front)
  const uint32_t kc0 = (dec ? wv : 0) * 32 + g * 8;
  const uint32_t grp = (uint32_t)((dec ? wv : 0) * 256) / (uint32_t)a.gsz_i;
  ScaleRaw sr[KMAX];
#pragma unroll
  for (int r = 0; r < KMAX; ++r) sr[r] = scale_raw(a.ds, a.sdt, (dbase[r] + j) * (uint32_t)a.Gi + grp);
  constexpr int PD = 3;
  uint4 q[KMAX];
  auto load_route = [&](int r) { q[r] = ldg16_q(a.dc + (size_t)(dbase[r] + j) * C + kc0); };
#pragma unroll
  for (int r = 0; r < PD && r < KMAX; ++r) load_route(r);
  const uint32_t rgrp = RES ? (uint32_t)((dec ? wv : 0) * 256) / (uint32_t)a.n.gsz_i : 0u;
  ScaleRaw srr[KMAX];
  uint2 qr[KMAX];
  if constexpr (RES) {  // residual scales and codes (C bytes per row), 2 KMAX more loads
#pragma unroll
    for (int r = 0; r < KMAX; ++r) srr[r] = scale_raw(a.n.ds, a.n.sdt, (rres[r] + j) * (uint32_t)a.n.Gi + rgrp);
#pragma unroll
    for (int r = 0; r < KMAX; ++r)
      qr[r] = res_load8(a.n.dc + (size_t)rres[r] * C, hot[r] && dec ? 16u * C : 0u, j * C + kc0);
  }
  __builtin_amdgcn_sched_barrier(0);
  // the table DMAs and h loads, not the scales and codes. (The compiler hoists
  // the A-term maxima and, with LDS DMAs in flight beside register loads, can
  // only wait for all of them; issuing every code load before that wait
  // measured slower, so it is left there.)
  wait_vm_q<KMAX + (PD < KMAX ? PD : KMAX) + (RES ? 2 * KMAX : 0)>();

  // 3. A terms: rows 2r, 2r + 1 of route r, scaled by the route's own power of two
  float inv4s[KMAX];
  {
    uint32_t* aw = (uint32_t*)ash;
#pragma unroll
    for (int r = 0; r < KMAX; ++r) {
      float v[4];
      q8_half4<true>(hq[r], lane & 1, v);
      const float mx = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
      float s;
      q8_scale(rt_wave_reduce(mx, true), s, inv4s[r]);
      uint32_t tw[2];
      q8_digits2(v, s, tw);
      aw[q8_aword((uint32_t)(wv * 2 * KMAX + 2 * r), lane >> 1, lane & 1)] = tw[0];
      aw[q8_aword((uint32_t)(wv * 2 * KMAX + 2 * r + 1), lane >> 1, lane & 1)] = tw[1];
    }
  }
  rt_lds_barrier();  // the table and A terms visible

  if (dec) {
    q8v4 A[4];
    {
      const bool live = j < 2u * KMAX;
      const q8v4* as = (const q8v4*)ash + (wv * 2 * KMAX + (live ? j : 0u)) * 16 + g * 4;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const q8v4 v = as[i];
        A[i] = live ? v : q8v4{0, 0, 0, 0};
      }
    }

    // 4. decode route by route
#pragma unroll
    for (int r = 0; r < KMAX; ++r) {  // branch-free: zero-weight routes are dropped in the sum
      if (r + PD < KMAX) load_route(r + PD);
      __builtin_amdgcn_sched_barrier(0);
      q8v4 B[4];
      q8_decode8(tq, lk, q[r], B);
      q8v4 acc = {0, 0, 0, 0};
#pragma unroll
      for (int i = 0; i < 4; ++i) acc = mfma_i8(A[i], B[i], acc);
      float vr = 0.f;
      if constexpr (RES) {
        if (hot[r]) {  // block-uniform
          q8v4 R[4];
          t8_decode8((const char*)t8s, (uint32_t)lane, qr[r], R);
          q8v4 accr = {0, 0, 0, 0};
#pragma unroll
          for (int i = 0; i < 4; ++i) accr = mfma_i8(A[i], R[i], accr);
          const float dr = (r & 1) ? (float)accr[2] + (float)accr[3] * 0.0078125f
                                   : (float)accr[0] + (float)accr[1] * 0.0078125f;
          vr = dr * inv4s[r] * scale_cvt(srr[r], a.n.sdt, (rres[r] + j) * (uint32_t)a.n.Gi + rgrp);
        }
      }
      // rows 2r, 2r + 1 live in lanes 16 (r / 2) + j, registers 2 (r % 2), 2 (r % 2) + 1
      if (g == (uint32_t)(r >> 1)) {
        const float d = (r & 1) ? (float)acc[2] + (float)acc[3] * 0.0078125f
                                : (float)acc[0] + (float)acc[1] * 0.0078125f;
        red[wv][r][j] = d * inv4s[r] * scale_cvt(sr[r], a.sdt, (dbase[r] + j) * (uint32_t)a.Gi + grp) + vr;
      }
    }
  }
  rt_lds_barrier();

  // 5. weighted sum over routes and waves
  if (threadIdx.x < 16) {
    float o = 0.f;
#pragma unroll
    for (int r = 0; r < KMAX; ++r) {
      float v = 0.f;
      for (int w = 0; w < nwd; ++w) v += red[w][r][threadIdx.x];
      o = wt[r] != 0.f ? fmaf(wt[r], v, o) : o;
    }
    if (bad || tq_bad) o = __builtin_nanf("");
    const size_t oi = n0 + threadIdx.x;
    if (a.odt == KEEP_F16) ((_Float16*)a.out)[oi] = (_Float16)o;
    else if (a.odt == KEEP_BF16) ((uint16_t*)a.out)[oi] = from_float<bf16s>(o).bits;
    else ((float*)a.out)[oi] = o;
  }
  wait_vm_q<0>();  // no DMA into this block's LDS may outlive it
}

// ------------------------------------------------------------------ host


void tq_build(const uint32_t* table, void* prepared, hipStream_t s) {
  hipLaunchKernelGGL(k_build_tq, dim3(1), dim3(256), 0, s, table, (uint2*)((char*)prepared + TQ_OFFSET),
                     (uint4*)((char*)prepared + TQR_OFFSET), (uint32_t*)((char*)prepared + TQ_FLAG_OFFSET));
}

bool moe_q_layer_supported(int64_t E, int64_t H, int64_t I, int64_t k, int64_t group_h, int64_t group_i) {
  if (!(H == 4096 && I >= 512 && I % 512 == 0 && I <= 2048 && k >= 1 && k <= 8 && k <= E && E <= 1024))
    return false;  // bounds first: the products below stay small
  const int64_t qtiles = k * I / 16;
  return (qtiles + 255) / 256 <= 3 && group_h >= 256 && group_h % 256 == 0 && group_i >= 256 &&
         group_i % 256 == 0;
}

void moe_q_down_launch(const int32_t* idx, const float* w, int64_t k, int64_t E, int64_t H, int64_t I,
                       const uint16_t* dc, const void* ds, int sdt, int64_t group_i, const void* prepared,
                       const void* h, void* out, int odt, hipStream_t s, const MQNest* nest) {
  MQDown d{};
  d.H = (int32_t)H; d.E = (int32_t)E; d.dc = dc; d.ds = ds; d.sdt = sdt;
  d.Gi = (int32_t)(I / group_i); d.gsz_i = (int32_t)group_i;
  d.tq_bad = (const uint32_t*)((const char*)prepared + TQ_FLAG_OFFSET);
  d.out = out; d.odt = odt;
  const uint4* tqr = (const uint4*)((const char*)prepared + TQR_OFFSET);
  const uint16_t* hin = (const uint16_t*)h;
  const int32_t Ii = (int32_t)I;
  if (nest) d.n = *nest;
  const dim3 grid((unsigned)(H / 16)), blk(512u);
#define DN(K)                                                                        \
  if (nest) hipLaunchKernelGGL((k_moeq_down<K, true>), grid, blk, 0, s, idx, w, tqr, hin, Ii, d); \
  else hipLaunchKernelGGL((k_moeq_down<K, false>), grid, blk, 0, s, idx, w, tqr, hin, Ii, d)
  switch (k) {
    case 1: DN(1); break;
    case 2: DN(2); break;
    case 3: DN(3); break;
    case 4: DN(4); break;
    case 5: DN(5); break;
    case 6: DN(6); break;
    case 7: DN(7); break;
    default: DN(8); break;
  }
#undef DN
}

int moe_q_layer_launch(const float* logits, const float* bias_s, const float* bias_d, int func, int renorm,
                       float route_scale, float tau, const int32_t* slot_map, int64_t S, int64_t E, int64_t k,
                       const void* x, int x_dtype, int64_t H,
                       int64_t I, const uint16_t* gc, const void* gs, const uint16_t* uc, const void* us,
                       const uint16_t* dc, const void* ds, int sdt, int64_t group_h, int64_t group_i,
                       const void* prepared, float limit, int32_t* idx, float* w, int32_t* want, float* want_score,
                       uint8_t* admit, void* h, void* out, int odt, hipStream_t s, const MQNest* nest) {
  MQLayer a{};
  a.func = func; a.renorm = renorm;
  a.same_bias = bias_s == bias_d; a.route_scale = route_scale; a.tau = tau; a.k = (int32_t)k;
  a.slot_map = slot_map; a.S = (int32_t)(slot_map ? S : E);
  a.idx_out = idx; a.w_out = w; a.want_out = want; a.want_score_out = want_score; a.admit_out = admit;
  a.H = (int32_t)H; a.I = (int32_t)I; a.gc = gc; a.uc = uc; a.gs = gs; a.us = us;
  a.sdt = sdt; a.Gh = (int32_t)(H / group_h); a.gsz_h = (int32_t)group_h;
  const uint4* tqr = (const uint4*)((const char*)prepared + TQR_OFFSET);
  a.tq_bad = (const uint32_t*)((const char*)prepared + TQ_FLAG_OFFSET);
  a.limit = limit; a.h = (uint16_t*)h;
  const int32_t Ei = (int32_t)E;
  a.qtiles = (int32_t)(k * I / 16);
  if (nest) a.n = *nest;
  const int qt = (int)((a.qtiles + 255) / 256);
  const dim3 grid((unsigned)((a.qtiles + qt - 1) / qt)), blk(1024);
#define LY(NT, BF, PER)                                                                    \
  if (nest)                                                                                    \
    hipLaunchKernelGGL((k_moeq_route_gateup<NT, BF, PER, true>), grid, blk, 0, s, logits, bias_s, bias_d, tqr, x, \
                       Ei, a);                                                                    \
  else                                                                                         \
    hipLaunchKernelGGL((k_moeq_route_gateup<NT, BF, PER, false>), grid, blk, 0, s, logits, bias_s, bias_d, tqr, x, \
                       Ei, a)
#define LY_PER(NT, BF)                 \
  if (E <= 256) LY(NT, BF, 4);         \
  else if (E <= 384) LY(NT, BF, 6);    \
  else if (E <= 512) LY(NT, BF, 8);    \
  else LY(NT, BF, 16)
#define LY_NT(BF) \
  if (qt <= 1) { LY_PER(2, BF); } else if (qt == 2) { LY_PER(4, BF); } else { LY_PER(6, BF); }
  if (x_dtype == KEEP_BF16) { LY_NT(true); } else { LY_NT(false); }
#undef LY_NT
#undef LY_PER
#undef LY
  moe_q_down_launch(idx, w, k, a.S, H, I, dc, ds, sdt, group_i, prepared, h, out, odt, s, nest);
  return 0;
}

// The residual LDS image (t8_entry per packed E8 entry, sixteen copies).
__global__ __launch_bounds__(256) void k_build_t8(const uint32_t* packed, uint2* image) {
  const uint32_t i = threadIdx.x;
  const uint2 v = t8_entry(packed[i]);
#pragma unroll
  for (int c = 0; c < 16; ++c) image[i * 16 + c] = v;
}

}  // namespace keep

using namespace keep;

extern "C" int keep_e8_1bit_image(const uint32_t* packed_table, void* image, void* stream) {
  KEEP_REQUIRE(packed_table && image, "table and image must be non-null");
  KEEP_REQUIRE(aligned(image, 16), "image must be 16-byte aligned");
  hipLaunchKernelGGL(k_build_t8, dim3(1), dim3(256), 0, (hipStream_t)stream, packed_table, (uint2*)image);
  return launch_status("keep_e8_1bit_image");
}

extern "C" int keep_e8_1bit_image_bytes(void) { return T8R_BYTES; }

extern "C" int keep_moe_layer_nested(
    const float* logits, const float* bias_served, const float* bias_demand, int score_func, int renormalize,
    float route_scale, float tau, const int32_t* slot_map, int64_t num_slots, int64_t E, int64_t k, const void* x,
    int x_dtype, int64_t H, int64_t I,
    const uint16_t* gate_codes, const void* gate_scales, const uint16_t* up_codes, const void* up_scales,
    const uint16_t* down_codes, const void* down_scales, int scale_dtype, int64_t group_size_h, int64_t group_size_i,
    const void* prepared, float swiglu_limit, int32_t* idx, float* w, int32_t* want, float* want_score,
    uint8_t* admit, void* h_work, void* out, int out_dtype, const uint32_t* hot_of_slot, int64_t num_hot,
    const uint8_t* res_gate_codes, const void* res_gate_scales, const uint8_t* res_up_codes,
    const void* res_up_scales, const uint8_t* res_down_codes, const void* res_down_scales, int res_scale_dtype,
    int64_t res_group_size_h, int64_t res_group_size_i, const void* res_image, int32_t* hot_route, void* stream) {
  KEEP_REQUIRE_DIMS(num_slots, E, k, H, I, group_size_h, group_size_i, num_hot, res_group_size_h, res_group_size_i);
  KEEP_REQUIRE(x_dtype == KEEP_F16 || x_dtype == KEEP_BF16, "activations must be fp16 or bf16");
  KEEP_REQUIRE(dtype_ok(scale_dtype) && dtype_ok(out_dtype) && dtype_ok(res_scale_dtype), "bad dtype enum");
  KEEP_REQUIRE(score_func >= 0 && score_func <= 2, "bad score_func %d", score_func);
  KEEP_REQUIRE(group_size_h > 0 && H % group_size_h == 0 && group_size_i > 0 && I % group_size_i == 0,
               "bad group sizes");
  KEEP_REQUIRE(!slot_map || (num_slots >= 1 && num_slots <= 1024), "num_slots must be in 1..1024");
  KEEP_REQUIRE(moe_q_layer_supported(E, H, I, k, group_size_h, group_size_i),
               "shape not served by the routed decode layer kernels (needs H = 4096, I a multiple of 512 up to "
               "2048, k <= 8, E <= 1024, scale groups of 256-element multiples)");
  KEEP_REQUIRE(res_group_size_h > 0 && H % res_group_size_h == 0 && res_group_size_h % 256 == 0 &&
                   res_group_size_i > 0 && I % res_group_size_i == 0 && res_group_size_i % 256 == 0,
               "residual scale groups must divide H and I and be multiples of 256");
  KEEP_REQUIRE(num_hot >= 1 && num_hot * I * H < (int64_t(1) << 31), "bad residual row count %lld",
               (long long)num_hot);
  KEEP_REQUIRE(logits && x && gate_codes && gate_scales && up_codes && up_scales && down_codes && down_scales &&
                   prepared && idx && w && h_work && out && hot_of_slot && res_gate_codes && res_gate_scales &&
                   res_up_codes && res_up_scales && res_down_codes && res_down_scales && res_image && hot_route,
               "null pointer argument");
  KEEP_REQUIRE(aligned(x, 16) && aligned(h_work, 16) && aligned(prepared, 16) && aligned(res_image, 16),
               "x, h_work, prepared and res_image must be 16-byte aligned");
  KEEP_REQUIRE(aligned(gate_codes, 16) && aligned(up_codes, 16) && aligned(down_codes, 8), "codes misaligned");
  KEEP_REQUIRE(aligned(res_gate_codes, 8) && aligned(res_up_codes, 8) && aligned(res_down_codes, 8) &&
                   aligned(hot_of_slot, 4) && aligned(hot_route, 4),
               "residual codes must be 8-byte aligned");
  MQNest n{};
  n.hot = (const int32_t*)hot_of_slot; n.nhot = (int32_t)num_hot;
  n.gc = res_gate_codes; n.uc = res_up_codes; n.dc = res_down_codes;
  n.gs = res_gate_scales; n.us = res_up_scales; n.ds = res_down_scales; n.sdt = res_scale_dtype;
  n.Gh = (int32_t)(H / res_group_size_h); n.gsz_h = (int32_t)res_group_size_h;
  n.Gi = (int32_t)(I / res_group_size_i); n.gsz_i = (int32_t)res_group_size_i;
  n.t8 = (const uint4*)res_image; n.hot_route = hot_route;
  moe_q_layer_launch(logits, bias_served, bias_demand, score_func, renormalize, route_scale, tau, slot_map,
                     num_slots, E, k, x, x_dtype,
                     H, I, gate_codes, gate_scales, up_codes, up_scales, down_codes, down_scales, scale_dtype,
                     group_size_h, group_size_i, prepared, swiglu_limit, idx, w, want, want_score, admit, h_work,
                     out, out_dtype, (hipStream_t)stream, &n);
  return launch_status("keep_moe_layer_nested");
}
