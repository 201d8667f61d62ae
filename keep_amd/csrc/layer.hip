// The routed MoE decode layer for one token in ONE launch on gfx950: dual
// top-k router, gate/up + SwiGLU, down + weighted combine. One block per
// CU (256 blocks of 16 waves, all resident together); block b owns three
// 16-row gate/up tiles of the [k, I] intermediate and the 16 output rows
// 16 b .. 16 b + 15 of down. The int8 decode of E8P codewords and the
// activation term split are described in q8_dev.h.
//
// As soon as a block has routed the token it issues the loads of its gate/up
// tiles; each wave issues its down rows (every route's 16 rows x the wave's
// 256-wide K slice) once its gate/up codes are in, so down's 12.6 MB stream
// behind gate/up's 25.2 MB with no kernel boundary and no second routing
// read. Gate/up decode and MFMAs run as their codes land; the block's SwiGLU
// outputs h are published, and down waits only for the h slices its waves
// consume.
//
// The h exchange. Blocks on different XCDs have different L2s, so h is
// exchanged through agent-scope atomic stores and loads (written through to,
// and read back from, the memory side of the L2s), with no fences and no
// cache flush. Each 64-bit word carries two bf16 h values and a 32-bit tag,
// the call's epoch + 1: a reader knows a word is this call's by its tag,
// word by word, so no flag has to be ordered after the data. The epoch lives
// in the caller's workspace (zero-filled before its first use): every block
// reads it at its start and then counts itself in; the last block to count
// in (so every block has read it) advances it for the next call. A wait that
// outlasts spin_ticks of the 100 MHz real-time counter gives up: the routes
// of the waiting wave are NaN, and so are the outputs of its block (each sums
// every route), and the workspace's status word records it.
//
// The nested 3-bit tier (RES): a pool row with a residual row r (hot[row] in
// [0, nhot); -1 none, anything else makes its routes NaN) adds the 8-bit E8
// residual r of gate, up and down (codes uint8 [nhot, N, K / 8], one byte per
// codeword indexing the packed E8 table; weight x 4 = 2 (nibble - 8), exact in
// int8) to its base: multiplied by the same A operands into a second
// accumulator and added, each with its own scale, before the SwiGLU and
// before the weighted sum (omlx_lattice.py:172-186, 358-370). Every block
// builds a 4-copy LDS image of the table (8 KiB; lane l reads copy l % 4).
#include <hip/hip_runtime.h>

#include <atomic>

#include "common.h"
#include "moe_dev.h"
#include "q8_dev.h"
#include "route_dev.h"

namespace keep {

constexpr int FL_BLOCKS = 256;       // H / 16 down row tiles, one block per CU
constexpr int FL_WAVES = 16;         // H / 256 gate/up K slices
constexpr uint32_t FL_HDR_BYTES = 256;  // epoch, arrivals, status
constexpr uint32_t FL_TIMEOUT = 1u;     // status bit: a wait gave up
constexpr uint32_t FL_CERT = 2u;        // status bit: a certified early route differed from the exact one
constexpr uint32_t FL_SPIN_TICKS_DEFAULT = 20000u;   // 200 us of the 100 MHz counter
constexpr uint32_t FL_SPIN_TICKS_MAX = 100000000u;   // 1 s

// The arguments the first loads need: the kernel's leading arguments,
// preloaded into SGPRs by the dispatcher (-amdgpu-kernarg-preload-count).
struct FLHead {
  const float* logits;
  const float *bias_s, *bias_d;
  const uint2* tq;  // T[256] then M[256], 8 bytes each (keep_e8p_prepare)
  const void* x;
  uint32_t* hdr;    // [0] epoch, [1] arrivals, [2] status
  int32_t E;
};

// The rest.
struct FLArgs {
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
  int xbf;  // x is bf16 (else fp16)
  int32_t I;
  const uint16_t *gc, *uc, *dc;
  const void *gs, *us, *ds;
  int sdt;
  int32_t Gh, gsz_h, Gi, gsz_i;
  const uint32_t* tq_bad;
  float limit;
  int32_t qtiles;
  uint64_t* hx;       // [k * I / 2] tagged h pairs
  uint32_t spin_ticks;
  void* out;
  int odt;
  // the nested tier (RES)
  const int32_t* hot;  // [S] residual row of each pool row
  int32_t nhot;
  const uint8_t *rgc, *ruc, *rdc;  // residual codes [nhot][N][K / 8]
  const void *rgs, *rus, *rds;
  int rsdt;
  int32_t rGh, rgsz_h, rGi, rgsz_i;
  const uint32_t* t8;  // the packed 8-bit E8 table, uint32[256]
};

// The residual image: entry n (the 8 bytes 2 (nibble d - 8), packed-nibble
// order) in four copies, copy c at n * 32 + 8 c; lane l reads copy l % 4.
constexpr int FL_T8_BYTES = 256 * 32;
__device__ __forceinline__ q8v4 fl_t8_decode2(const char* img, uint32_t lane, uint32_t w) {
  const uint32_t c8 = (lane & 3u) * 8u;
  const uint2 x0 = *(const uint2*)(img + (w & 0xffu) * 32u + c8);
  const uint2 x1 = *(const uint2*)(img + ((w >> 8) & 0xffu) * 32u + c8);
  return q8v4{(int)x0.x, (int)x0.y, (int)x1.x, (int)x1.y};
}
// B operands of 8 residual code bytes (codewords 2i, 2i + 1 -> R[i]).
__device__ __forceinline__ void fl_t8_decode8(const char* img, uint32_t lane, uint2 q, q8v4 (&R)[4]) {
  R[0] = fl_t8_decode2(img, lane, q.x);
  R[1] = fl_t8_decode2(img, lane, q.x >> 16);
  R[2] = fl_t8_decode2(img, lane, q.y);
  R[3] = fl_t8_decode2(img, lane, q.y >> 16);
}

__device__ __forceinline__ uint64_t fl_load(const uint64_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void fl_store(uint64_t* p, uint64_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Position of dim d (0..7) inside a codeword's 8 values in packed-nibble
// order (dims 0, 2, 4, 6, 1, 3, 5, 7), the order the A operands use.
__device__ __forceinline__ uint32_t fl_pos(uint32_t d) { return (d & 1u) * 4u + (d >> 1); }

// NT gate/up tiles per block (two per 16-row q-tile), PER logits per router
// lane, NSL = I / 256 down K slices, RPW routes per down wave (RG = 16 / NSL
// route groups of RPW routes: the waves w < NSL * RG own slice w % NSL and
// route group w / NSL). G1: per-row gate and up scales (one scale group per
// row), applied once to each row's sum instead of to every slice's partial;
// with RES the residual's gate and up scales are per row as well, and each
// wave keeps its residual partials apart (in its own slice of the x-term
// LDS, free once the wave holds its A operands) for the same fold.
//
// LDS is one array with the decode image at address 0, so a lookup address
// is exactly the byte permute of q8_decode2 (no base to add).
template <int NT, int PER, int NSL, int RPW, bool G1, bool RES>
__global__ __launch_bounds__(1024) void k_moe_layer1(const float* logits, const float* bias_s, const float* bias_d,
                                                     const uint2* tqe, const void* xin, uint32_t* hdr, int32_t E,
                                                     FLArgs a) {
  constexpr int QT = NT / 2;
  constexpr int RG = FL_WAVES / NSL;
  static_assert(RPW * 4 <= 16, "at most four routes per down wave (A rows 4 r + t)");
  constexpr int O_DSH = TQR_BYTES;                      // down terms [wave][row 4 r + t][g * 4 + i]
  constexpr int O_ASH = O_DSH + FL_WAVES * 16 * 256;    // x terms [slice][term][g * 4 + i]
  constexpr int O_GRED = O_ASH + 16 * 3 * 256;          // gate/up partials [wave][tile][row]
  constexpr int O_RED = O_GRED + 16 * NT * 16 * 4;      // down partials [row][wave]
  constexpr int O_SMALL = O_RED + 16 * 16 * 4;         // s_inv4s[16], s_idx[8], s_w[8], s_hr[8], s_cert, s_chk
  constexpr int O_T8 = O_SMALL + 256;                   // RES: the residual image
  constexpr int LDS_BYTES = O_T8 + (RES ? FL_T8_BYTES : 0);
  __shared__ uint4 smem[LDS_BYTES / 16];
  char* lds = (char*)smem;
  uint4* tqs = smem;
  uint4* dsh = (uint4*)(lds + O_DSH);
  uint4* ash = (uint4*)(lds + O_ASH);
  float* gred = (float*)(lds + O_GRED);
  float* gres = (float*)(lds + O_ASH);  // RES and G1: wave w's residual partials [tile][row] at float w * 192 (its x-term slice)
  float* red = (float*)(lds + O_RED);
  float* s_inv4s = (float*)(lds + O_SMALL);
  int32_t* s_idx = (int32_t*)(lds + O_SMALL + 64);
  float* s_w = (float*)(lds + O_SMALL + 96);
  int32_t* s_hr = (int32_t*)(lds + O_SMALL + 128);  // RES: each route's residual row (-1 none, -2 invalid)
  int32_t* s_cert = (int32_t*)(lds + O_SMALL + 160);  // the block's routing state (lds_flag)
  int32_t* s_chk = (int32_t*)(lds + O_SMALL + 164);
  const char* t8i = lds + O_T8;
  const char* tq = (const char*)tqs;
  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const Q8Keys lk = q8_keys((uint32_t)lane);
  const uint32_t j = lane & 15, g = lane >> 4;
  const uint32_t C = 4096u >> 3;  // H / 8 token chunks
  const uint32_t CI = (uint32_t)a.I >> 3;
  const uint32_t b = blockIdx.x;

  // 0. the call's epoch; the router's inputs (waves 0 and 1); T and M for the
  //    image (every thread builds four copies of one entry); the token slices
  //    this wave builds terms for (wave w >= 2 slice w; waves 2 and 3 also
  //    slices 0 and 1), all from the preloaded arguments; then the table flag
  //    and the slot map, which need the others
  const uint32_t ep_word = __hip_atomic_load(hdr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  float z[PER], bsv[PER], bdv[PER];
  int sm[PER];
  if (wv < 2) rt_load<PER>(logits, bias_s, bias_d, E, lane, z, bsv, bdv);
  const uint32_t te = threadIdx.x >> 2;
  const uint2 tv = tqe[te], mv = tqe[256 + te];
  const uint4 xc = ldg16_q((const uint4*)xin + (wv < 2 ? 0 : wv) * 32 + (lane >> 1));
  const uint4 xc2 = ldg16_q((const uint4*)xin + (wv < 4 ? (wv & 1) : 0) * 32 + (lane >> 1));
  __builtin_amdgcn_sched_barrier(0);
  const uint32_t tq_bad = ((const __attribute__((address_space(4))) uint32_t*)a.tq_bad)[0];
  if (wv < 2 && a.slot_map) rt_load_slots<PER>(a.slot_map, E, lane, sm);
  int hv[PER];  // RES: the residual rows of pool rows lane + 64 i (waves 0 and 1)
  uint32_t t8w = 0u;
  if constexpr (RES) {
    if (wv < 2) rt_load_slots<PER>(a.hot, a.S, lane, hv);
    t8w = a.t8[threadIdx.x >> 2];
  }
  __builtin_amdgcn_sched_barrier(0);
  const uint32_t ep = __builtin_amdgcn_readfirstlane(ep_word);
  {
    // the four threads of entry te write its sixteen copies; store k of thread
    // (te, c) takes copy (4 c + te + k) & 15, so the sixteen lanes of an LDS
    // pass (four entries x four threads) write sixteen different copies, each
    // a distinct group of four banks
    const uint4 v = make_uint4(tv.x, tv.y, mv.x, mv.y);
    uint4* row = tqs + te * 16;
    const uint32_t c0 = (threadIdx.x & 3) * 4 + te;
#pragma unroll
    for (uint32_t k = 0; k < 4; ++k) row[(c0 + k) & 15u] = v;
    if constexpr (RES) *(uint2*)(lds + O_T8 + (threadIdx.x >> 2) * 32 + (threadIdx.x & 3) * 8) = t8_entry(t8w);
  }
  // RES: the residual row of pool row `slot` (a routing wave, every lane takes part): -1 none, -2 invalid
  auto hot_of = [&](int slot) -> int {
    const bool in = slot >= 0 && slot < a.S;
    const int ss = in ? slot : 0, owner = ss & 63, i0 = ss >> 6;
    int v = -1;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int x = __shfl(hv[i], owner, 64);
      v = i == i0 ? x : v;
    }
    return !in || v == -1 ? -1 : (v >= 0 && v < a.nhot ? v : -2);
  };

  // 1. routing. The selection order is "larger key, then lower index" over the
  //    keys score + bias. Every score function is increasing in the logit, so
  //    where each bias is 0 or at most RT_MASKED (no bias, or the residency
  //    mask) the logits order the unmasked experts as the keys do and the bias
  //    values order the masked ones, except where the score rounding makes two
  //    keys equal whose logits differ. Wave 0 selects the routes of this
  //    block's gate/up tiles (0 .. kneed - 1) on those logit keys, without the
  //    score function, and the tiles' loads issue on them. For the softmax it
  //    also certifies them: with every logit finite and each selected route's
  //    logit at least 2^-16 above the next one's, within 60 of the largest
  //    logit, the softmax keys are strictly ordered the same way (the
  //    difference z - m rounds by at most 2^-17, the exponential then differs
  //    by a factor above 1 + 2^-18 and the division keeps that order). Wave 1
  //    forms the exact selection of all k routes meanwhile (the later routes,
  //    the weights and the outputs); when wave 0 could not certify, every wave
  //    waits for it before its first decode and reloads its tiles if an early
  //    route differed. With other biases wave 0 selects on the exact keys.
  //    A terms: rows 0-2 of slice w are the three int8 terms of x s, s the
  //    slice's power of two (waves >= 2, meanwhile).
  float sc[PER];
  int e_sel = -1, sl = -1;
  const int qlast = min((int)(b * QT + QT - 1), a.qtiles - 1);
  const int kneed = qlast < (int)(b * QT) ? 1 : min(a.k, qlast * 16 / a.I + 1);
  RtSel<PER> sel;
  bool certify = false;  // wave 0: the softmax of finite logits under plain biases
  auto build = [&](uint4 c, int slice) {
    float v[4];
    if (a.xbf) q8_half4<true>(c, lane & 1, v);
    else q8_half4<false>(c, lane & 1, v);
    float mx = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
    float s, inv4s;
    q8_scale(rt_wave_max_abs(mx), s, inv4s);
    uint32_t tw[3];
    q8_terms<3>(v, s, tw);
    uint32_t* aw = (uint32_t*)ash;
#pragma unroll
    for (int n = 0; n < 3; ++n) aw[q8_aword((uint32_t)(slice * 3 + n), lane >> 1, lane & 1)] = tw[n];
    if (lane == 0) s_inv4s[slice] = inv4s;
  };
  // the block's routing state in LDS, read wave-uniform: s_cert (wave 0) 1 the
  // early routes are certified, 2 not; s_chk (wave 1) bit 1 every route is in
  // s_idx / s_hr, bit 0 an early route differed from the exact one. Both are
  // zeroed before the first barrier and set after it.
  auto lds_flag = [&](int32_t* f) -> int {
    return __builtin_amdgcn_readfirstlane(__hip_atomic_load(f, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP));
  };
  auto slot_of = [&](int e) -> int {
    return a.slot_map ? rt_slot_of<PER>(sm, e, E, a.S) : (e >= 0 && e < E ? e : -1);
  };
  if (wv == 0) {
    bool plain = true, finite = true;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      plain = plain && (bsv[i] == 0.f || bsv[i] <= RT_MASKED);
      finite = finite && (lane + 64 * i >= E || fabsf(z[i]) < __builtin_inff());
    }
    uint32_t kk[PER];
    const bool proxy = __all(plain);
    if (proxy) {
#pragma unroll
      for (int i = 0; i < PER; ++i) kk[i] = lane + 64 * i < E ? rt_sortable(bsv[i] != 0.f ? bsv[i] : z[i]) : 0u;
    } else {
      rt_scores<PER>(z, E, a.func, lane, sc);
      rt_keys<PER>(sc, bsv, E, lane, kk);
    }
    sel.init(kk, lane);
    sel.rounds(0, kneed, lane, 0);
    sl = slot_of(sel.mine);
    if (lane < kneed) s_idx[lane] = sl;
    if constexpr (RES) {
      const int hr = hot_of(sl);
      if (lane < kneed) s_hr[lane] = hr;
    }
    certify = proxy && a.func == KEEP_SCORE_SOFTMAX && __all(finite);
    if (lane == 0) *s_cert = 0;
  } else if (wv == 1) {
    rt_scores<PER>(z, E, a.func, lane, sc);
    if (lane == 0) *s_chk = 0;
  } else {
    build(xc, wv);
    if (wv < 4) build(xc2, wv - 2);
  }
  rt_lds_barrier();  // the routes of the tiles' loads in s_idx, the image and every slice's A terms

  // 2. the gate/up loads of the block: scales and codes
  uint32_t rbase[QT];
  const uint32_t grp = G1 ? 0u : (uint32_t)(wv * 256) / (uint32_t)a.gsz_h;
  const uint32_t kc0 = wv * 32 + g * 8;
  ScaleRaw sr[NT];
  uint4 q[NT];
  int hrt[QT];
  uint32_t rrow[QT];
  uint2 qr[NT];
  ScaleRaw srr[NT];
  const uint32_t rgrp = RES ? (uint32_t)(wv * 256) / (uint32_t)a.rgsz_h : 0u;
  auto issue = [&]() {
#pragma unroll
    for (int u = 0; u < QT; ++u) {
      const uint32_t qt = b * QT + u;
      const bool valid = qt < (uint32_t)a.qtiles;
      const uint32_t q0 = (valid ? qt : 0u) * 16u;
      const uint32_t route = q0 / (uint32_t)a.I;
      const int32_t e = s_idx[route];
      const bool ok = valid && e >= 0 && e < a.S;
      rbase[u] = (ok ? (uint32_t)e * (uint32_t)a.I : 0u) + (q0 - route * (uint32_t)a.I);
    }
    // G1: the row scales of the reducing lanes (wave 0, lane 16 u + jj: row jj of q-tile u); else every
    // wave's slice scales
    if constexpr (G1) {
      uint32_t rb = rbase[0];
#pragma unroll
      for (int u = 1; u < QT; ++u) rb = (lane >> 4) == (uint32_t)u ? rbase[u] : rb;
      const uint32_t si = rb + j;
      sr[0] = wv == 0 && lane < QT * 16 ? scale_raw(a.gs, a.sdt, si) : 0u;
      sr[1] = wv == 0 && lane < QT * 16 ? scale_raw(a.us, a.sdt, si) : 0u;
    } else {
#pragma unroll
      for (int u = 0; u < QT; ++u) {
        const uint32_t si = (rbase[u] + j) * (uint32_t)a.Gh + grp;
        sr[2 * u] = scale_raw(a.gs, a.sdt, si);
        sr[2 * u + 1] = scale_raw(a.us, a.sdt, si);
      }
    }
    // the codes: every tile's 16 B per lane issued before any is needed
#pragma unroll
    for (int t = 0; t < NT; ++t)
      q[t] = ldg16_q(((t & 1) ? a.uc : a.gc) + (size_t)(rbase[t >> 1] + j) * C + kc0);
    // RES: each hot tile's residual codes (8 bytes per lane: codewords kc0 ..) and slice scales
    if constexpr (RES) {
#pragma unroll
      for (int u = 0; u < QT; ++u) {
        const uint32_t qt = b * QT + u;
        const bool valid = qt < (uint32_t)a.qtiles;
        const uint32_t q0 = (valid ? qt : 0u) * 16u;
        const uint32_t route = q0 / (uint32_t)a.I;
        hrt[u] = valid ? s_hr[route] : -1;
        rrow[u] = (hrt[u] >= 0 ? (uint32_t)hrt[u] * (uint32_t)a.I : 0u) + (q0 - route * (uint32_t)a.I);
      }
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        if (hrt[t >> 1] >= 0) {  // block-uniform
          qr[t] = ldg8_q(((t & 1) ? a.ruc : a.rgc) + (size_t)(rrow[t >> 1] + j) * C + kc0);
          if constexpr (!G1)
            srr[t] = scale_raw((t & 1) ? a.rus : a.rgs, a.rsdt, (rrow[t >> 1] + j) * (uint32_t)a.rGh + rgrp);
        } else {
          qr[t] = make_uint2(0u, 0u);
          if constexpr (!G1) srr[t] = 0u;
        }
      }
      if constexpr (G1) {  // the residual row scales of the reducing lanes (as sr)
        uint32_t rr = rrow[0];
        int hu = hrt[0];
#pragma unroll
        for (int u = 1; u < QT; ++u) {
          rr = (lane >> 4) == (uint32_t)u ? rrow[u] : rr;
          hu = (lane >> 4) == (uint32_t)u ? hrt[u] : hu;
        }
        const bool ld = wv == 0 && lane < QT * 16 && hu >= 0;
        srr[0] = ld ? scale_raw(a.rgs, a.rsdt, rr + j) : 0u;
        srr[1] = ld ? scale_raw(a.rus, a.rsdt, rr + j) : 0u;
      }
    }
  };
  if (wv == 0) {
    // the certificate: lane j < kneed compares its winner with winner j + 1
    // (a masked winner's key is its bias, <= RT_MASKED: no logit below it)
    bool sure = false;
    if (certify) {
      sel.rounds(kneed, min(kneed + 1, E), lane, 0);
      float m = -__builtin_inff();
#pragma unroll
      for (int i = 0; i < PER; ++i) m = fmaxf(m, z[i]);
      m = rt_wave_reduce(m, true);
      const float zj = rt_unsortable(sel.mine_key);
      const uint32_t kn = (uint32_t)__builtin_amdgcn_mov_dpp((int)sel.mine_key, 0x101, 0xF, 0xF, false);  // row_shl:1
      const float zn = rt_unsortable(kn);
      const bool next_masked = kn == 0u || zn <= RT_MASKED;
      const bool ok = next_masked || (zj - zn >= 0x1p-16f && zn >= m - 60.f);
      sure = __all(lane >= kneed || ok);
    }
    if (lane == 0) *s_cert = sure ? 1 : 2;
  }
  issue();
  __builtin_amdgcn_sched_barrier(0);
  if (wv == 1) {
    // the exact selection of every route, its check against wave 0's, the
    // residual rows, the served weights and outputs (a certified route equals
    // the exact one, so rewriting it changes nothing)
    uint32_t kk[PER];
    rt_keys<PER>(sc, bsv, E, lane, kk);
    sel.init(kk, lane);
    sel.rounds(0, a.k, lane, 0);
    e_sel = sel.mine;
    sl = slot_of(e_sel);
    const int early = lane < kneed ? s_idx[lane] : sl;
    const bool differ = __any(early != sl);
    if (lane < a.k) s_idx[lane] = sl;
    if constexpr (RES) {
      const int hr = hot_of(sl);
      if (lane < a.k) s_hr[lane] = hr;
    }
    if (lane == 0) *s_chk = differ ? 3 : 2;  // bit 1: every route is in s_idx / s_hr; bit 0: an early one differed
    const RouteLane r = rt_finish<PER>(e_sel, true, sc, bsv, E, a.k, lane, 0, a.renorm, a.route_scale, a.tau);
    if (lane < a.k) s_w[lane] = r.valid ? r.value : 0.f;
    if (b == 0 && r.valid) {
      a.idx_out[lane] = sl;  // the pool row (the expert itself without a slot map)
      a.w_out[lane] = r.value;
    }
  }
  {
    // the early routes are certified, or wave 1 has checked them (rare)
    int c = lds_flag(s_cert);
    while (c == 0) {
      __builtin_amdgcn_s_sleep(1);
      c = lds_flag(s_cert);
    }
    int f = c == 1 ? 0 : lds_flag(s_chk);
    while (c != 1 && !(f & 2)) {
      __builtin_amdgcn_s_sleep(1);
      f = lds_flag(s_chk);
    }
    if (f & 1) {  // block-uniform: an early route differed from the exact one
      issue();
      wait_vm_q<0>();  // every tile in before the decode, so the common path keeps exact wait counts
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

  // 3. gate/up, tile by tile as the codes land
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    q8v4 B[4];
    q8_decode8(tq, lk, q[t], B);
    q8v4 acc = {0, 0, 0, 0};
#pragma unroll
    for (int i = 0; i < 4; ++i) acc = mfma_i8(A[i], B[i], acc);
    float vres = 0.f;  // RES: the residual's scaled partial (G1: its unscaled partial, kept apart)
    if constexpr (RES) {
      if (hrt[t >> 1] >= 0) {  // block-uniform
        q8v4 R[4];
        fl_t8_decode8(t8i, (uint32_t)lane, qr[t], R);
        q8v4 accr = {0, 0, 0, 0};
#pragma unroll
        for (int i = 0; i < 4; ++i) accr = mfma_i8(A[i], R[i], accr);
        const float dr = ((float)accr[0] + (float)accr[1] * 0.0078125f) + (float)accr[2] * 0.00006103515625f;
        if constexpr (G1) {
          if (lane < 16) gres[wv * 192 + t * 16 + (int)j] = dr * inv4s;
        } else {
          vres = dr * inv4s * scale_cvt(srr[t], a.rsdt, (rrow[t >> 1] + j) * (uint32_t)a.rGh + rgrp);
        }
      }
    }
    if (lane < 16) {
      const float d = ((float)acc[0] + (float)acc[1] * 0.0078125f) + (float)acc[2] * 0.00006103515625f;
      if constexpr (G1) {
        gred[(wv * NT + t) * 16 + j] = d * inv4s;
      } else {
        const uint32_t si = (rbase[t >> 1] + j) * (uint32_t)a.Gh + grp;
        gred[(wv * NT + t) * 16 + j] = d * inv4s * scale_cvt(sr[t], a.sdt, si) + vres;
      }
    }
  }
  // down's loads, once this wave's gate/up codes are in (requested together
  // they would share the memory system with gate/up, which gates the exchange)
  __builtin_amdgcn_sched_barrier(0);
  // down: this wave's slice sd and routes rg * RPW + r' (every route written by wave 1 first)
  while (!(lds_flag(s_chk) & 2)) __builtin_amdgcn_s_sleep(1);
  const bool dwave = wv < NSL * RG;  // wave-uniform
  const int sd = dwave ? wv % NSL : 0, rg = dwave ? wv / NSL : 0;
  uint32_t dbase[RPW];
  bool dlive[RPW], dok[RPW];
#pragma unroll
  for (int r = 0; r < RPW; ++r) {
    const int route = rg * RPW + r;
    const int32_t e = route < a.k ? s_idx[route] : -1;
    dlive[r] = dwave && route < a.k;
    dok[r] = dlive[r] && e >= 0 && e < a.S;
    dbase[r] = (dok[r] ? (uint32_t)e * 4096u : 0u) + b * 16u;
  }
  const uint32_t dgrp = (uint32_t)(sd * 256) / (uint32_t)a.gsz_i;
  ScaleRaw srd[RPW];
#pragma unroll
  for (int r = 0; r < RPW; ++r) srd[r] = scale_raw(a.ds, a.sdt, (dbase[r] + j) * (uint32_t)a.Gi + dgrp);
  uint4 qd[RPW];
#pragma unroll
  for (int r = 0; r < RPW; ++r) qd[r] = ldg16_q(a.dc + (size_t)(dbase[r] + j) * CI + sd * 32 + g * 8);
  // RES: each hot route's residual down codes and slice scale
  int hrd[RPW];
  uint32_t drow[RPW];
  uint2 qrd[RPW];
  ScaleRaw srrd[RPW];
  const uint32_t rdgrp = RES ? (uint32_t)(sd * 256) / (uint32_t)a.rgsz_i : 0u;
  if constexpr (RES) {
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
      const int route = rg * RPW + r;
      hrd[r] = dok[r] ? s_hr[route] : -1;  // wave-uniform
      drow[r] = (hrd[r] >= 0 ? (uint32_t)hrd[r] * 4096u : 0u) + b * 16u;
      if (hrd[r] >= 0) {
        qrd[r] = ldg8_q(a.rdc + (size_t)(drow[r] + j) * CI + sd * 32 + g * 8);
        srrd[r] = scale_raw(a.rds, a.rsdt, (drow[r] + j) * (uint32_t)a.rGi + rdgrp);
      } else {
        qrd[r] = make_uint2(0u, 0u);
        srrd[r] = 0u;
      }
    }
  }
  // this block counts itself in (it has read the epoch); the last block in advances it after the exchange
  uint32_t arrived = 0u;
  if (threadIdx.x == 0)
    arrived = __hip_atomic_fetch_add(hdr + 1, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  rt_lds_barrier();  // every wave's partials (and s_w) visible

  // 4. SwiGLU of the block's rows and their publication: lane (u, jj) owns
  //    intermediate row 16 qt + jj; lanes with dim bit 1 clear publish the
  //    word of their dim and dim + 2 (adjacent in packed-nibble order)
  const uint32_t tag = ep + 1u;
  if (wv == 0 && lane < QT * 16) {
    const uint32_t u = lane >> 4, jj = lane & 15;
    const uint32_t qt = b * QT + u;
    float gsum = 0.f, usum = 0.f;
    for (int w = 0; w < 16; ++w) {
      gsum += gred[(w * NT + 2 * u) * 16 + jj];
      usum += gred[(w * NT + 2 * u + 1) * 16 + jj];
    }
    const bool valid = qt < (uint32_t)a.qtiles;
    const uint32_t q0 = (valid ? qt : 0u) * 16u;
    const int32_t e = s_idx[q0 / (uint32_t)a.I];
    if constexpr (G1) {
      uint32_t rb = rbase[0];
#pragma unroll
      for (int v = 1; v < QT; ++v) rb = u == (uint32_t)v ? rbase[v] : rb;
      gsum *= scale_cvt(sr[0], a.sdt, rb + jj);
      usum *= scale_cvt(sr[1], a.sdt, rb + jj);
      if constexpr (RES) {
        uint32_t rr = rrow[0];
        int hu = hrt[0];
#pragma unroll
        for (int v = 1; v < QT; ++v) {
          rr = u == (uint32_t)v ? rrow[v] : rr;
          hu = u == (uint32_t)v ? hrt[v] : hu;
        }
        if (hu >= 0) {
          float gr = 0.f, ur = 0.f;
          for (int w = 0; w < 16; ++w) {
            gr += gres[w * 192 + (int)(2 * u) * 16 + (int)jj];
            ur += gres[w * 192 + (int)(2 * u + 1) * 16 + (int)jj];
          }
          gsum += gr * scale_cvt(srr[0], a.rsdt, rr + jj);
          usum += ur * scale_cvt(srr[1], a.rsdt, rr + jj);
        }
      }
    }
    float hv = silu_mul(gsum, usum, a.limit);
    if (tq_bad || e < 0 || e >= a.S) hv = __builtin_nanf("");
    if (RES && s_hr[q0 / (uint32_t)a.I] == -2) hv = __builtin_nanf("");
    const uint32_t hb = from_float<bf16s>(hv).bits;
    const uint32_t hb2 = (uint32_t)__shfl((int)hb, lane ^ 2, 64);
    if (valid && (jj & 2u) == 0u) {
      const uint32_t i = q0 + jj;  // flat [k, I] index
      const uint32_t widx = ((i & ~7u) + fl_pos(i & 7u)) >> 1;
      fl_store(a.hx + widx, ((uint64_t)tag << 32) | hb | (hb2 << 16));
    }
  }

  // the demand routing's outputs (block 0, wave 1), recomputed from the
  // logits while the other blocks' h is awaited
  if (wv == 1 && b == 0 && (a.want_out || a.want_score_out || a.admit_out)) {
    float z1[PER], bs1[PER], bd1[PER], sc1[PER];
    rt_load<PER>(logits, bias_s, bias_d, E, lane, z1, bs1, bd1);
    const int d_sel = rt_select_pair<PER>(z1, bs1, bd1, E, a.k, a.func, a.same_bias != 0, 1, lane, sc1);
    const RouteLane r = rt_finish<PER>(d_sel, false, sc1, bs1, E, a.k, lane, 0, a.renorm, a.route_scale, a.tau);
    if (r.valid) {
      if (a.want_out) a.want_out[lane] = r.expert;
      if (a.want_score_out) a.want_score_out[lane] = r.value;
      if (a.admit_out) a.admit_out[lane] = r.admit;
    }
  }

  // 5. down: this wave's h slices (two words per lane and route: dims 2t +
  //    (lane & 1) of codeword lane / 2), waiting word by word for this call's tag
  if (dwave) {
    // down's B operands do not depend on h: decode them while h is awaited
    // (with four routes per wave all four would not fit in the registers:
    // the first two then, the other two once h is in)
    constexpr int NPRE = RPW <= 3 ? RPW : 2;
    q8v4 BD[RPW][4];
#pragma unroll
    for (int r = 0; r < NPRE; ++r) q8_decode8(tq, lk, qd[r], BD[r]);
    // every pass issues all of the wave's loads before it waits (a route
    // past k reads route 0's words and ignores them)
    const uint64_t* hp[RPW];
#pragma unroll
    for (int r = 0; r < RPW; ++r)
      hp[r] = a.hx + (((dlive[r] ? (uint32_t)(rg * RPW + r) : 0u) * (uint32_t)a.I + sd * 256u + lane * 4u) >> 1);
    uint64_t hw[RPW][2];
    const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
    bool gave_up = false;
    for (;;) {
#pragma unroll
      for (int r = 0; r < RPW; ++r)
#pragma unroll
        for (int h = 0; h < 2; ++h) hw[r][h] = fl_load(hp[r] + h);
      bool all = true;
#pragma unroll
      for (int r = 0; r < RPW; ++r)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          all = all && (!dlive[r] || (uint32_t)(hw[r][h] >> 32) == tag);
          if (!dlive[r]) hw[r][h] = 0u;
        }
      if (__all(all)) break;  // every lane holds every word
      if (__builtin_amdgcn_s_memrealtime() - t0 > a.spin_ticks) {
        gave_up = true;
        break;
      }
      __builtin_amdgcn_s_sleep(1);
    }
    if (gave_up && lane == 0) {
      __hip_atomic_fetch_or(hdr + 2, FL_TIMEOUT, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    // A terms: rows 4 r and 4 r + 1 of route r's slice, the two int8 digits
    // (base 256) of h s with s the slice's power of two, formed from the
    // slice's largest |h| on the scalar unit (a wave that gave up makes every
    // route it holds NaN)
    float inv4d[RPW];
    uint32_t* aw = (uint32_t*)(dsh + wv * 256);
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
      const uint32_t w0 = (uint32_t)hw[r][0], w1 = (uint32_t)hw[r][1];
      const float v[4] = {__uint_as_float(w0 << 16), __uint_as_float(w0 & 0xffff0000u), __uint_as_float(w1 << 16),
                          __uint_as_float(w1 & 0xffff0000u)};
      // max |h| by the bits: a NaN outranks every number and makes inv4d NaN
      const uint32_t a0 = w0 & 0x7fff7fffu, a1 = w1 & 0x7fff7fffu;
      const uint32_t m = max(max(a0 << 16, a0 & 0xffff0000u), max(a1 << 16, a1 & 0xffff0000u));
      float s;
      q8_scale(__uint_as_float(__builtin_amdgcn_readfirstlane(rt_wave_u32<true>(m))), s, inv4d[r]);
      if (gave_up) inv4d[r] = __builtin_nanf("");
      uint32_t tw[2];
      q8_digits2_b256(v, s * 256.f, tw);
#pragma unroll
      for (int n = 0; n < 2; ++n) aw[q8_aword((uint32_t)(4 * r + n), lane >> 1, lane & 1)] = tw[n];
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);  // this wave's LDS writes before its reads
    q8v4 AD[4];
    {
      const bool live = (j & 3u) < 2u && (int)(j >> 2) < RPW;
      const q8v4* as = (const q8v4*)aw + (live ? j : 0u) * 16 + g * 4;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const q8v4 v = as[i];
        AD[i] = live ? v : q8v4{0, 0, 0, 0};
      }
    }
    // route r's dot is D rows 4 r and 4 r + 1, held by lanes 16 r + jj; lane
    // (g, jj) keeps route g's weighted value for output row jj (NaN for a
    // route with a nonzero weight and no pool row, which makes the output NaN)
    float c = 0.f;
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
      if (r >= NPRE) q8_decode8(tq, lk, qd[r], BD[r]);
      q8v4 acc = {0, 0, 0, 0};
#pragma unroll
      for (int i = 0; i < 4; ++i) acc = mfma_i8(AD[i], BD[r][i], acc);
      float vres = 0.f;
      bool rbad = false;
      if constexpr (RES) {
        rbad = hrd[r] == -2;
        if (hrd[r] >= 0) {  // wave-uniform
          q8v4 R[4];
          fl_t8_decode8(t8i, (uint32_t)lane, qrd[r], R);
          q8v4 accr = {0, 0, 0, 0};
#pragma unroll
          for (int i = 0; i < 4; ++i) accr = mfma_i8(AD[i], R[i], accr);
          const float dr = (float)accr[0] + (float)accr[1] * 0.00390625f;
          vres = dr * inv4d[r] * scale_cvt(srrd[r], a.rsdt, (drow[r] + j) * (uint32_t)a.rGi + rdgrp);
        }
      }
      if ((int)g == r) {
        const int route = rg * RPW + r;
        const float wt = dlive[r] ? s_w[route] : 0.f;
        const float d = (float)acc[0] + (float)acc[1] * 0.00390625f;
        const float val = d * inv4d[r] * scale_cvt(srd[r], a.sdt, (dbase[r] + j) * (uint32_t)a.Gi + dgrp) + vres;
        c = wt == 0.f ? 0.f : (dok[r] && !rbad) ? wt * val : __builtin_nanf("");
      }
    }
    // the sum over the wave's routes (lane rows 0 + 1, then + rows 2 + 3)
    const auto p16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(c), __float_as_uint(c), false, false);
    c = __uint_as_float(p16[0]) + __uint_as_float(p16[1]);
    const auto p32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(c), __float_as_uint(c), false, false);
    c = __uint_as_float(p32[0]) + __uint_as_float(p32[1]);
    if (lane < 16) red[lane * 16 + wv] = c;
  } else if (lane < 16) {
    red[lane * 16 + wv] = 0.f;
  }
  if (threadIdx.x == 0 && arrived == FL_BLOCKS - 1) {  // every block has read the epoch: advance it
    __hip_atomic_store(hdr + 1, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(hdr, ep + 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  rt_lds_barrier();

  // 6. the sum of the waves' weighted partials, in wave order (a certified
  //    block whose exact routes differ would be a broken certificate: its
  //    outputs are NaN and the status word records it; never expected)
  const bool bad_cert = *s_cert == 1 && (*s_chk & 1);
  if (bad_cert && threadIdx.x == 0)
    __hip_atomic_fetch_or(hdr + 2, FL_CERT, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (threadIdx.x < 16) {
    const float4* rp = (const float4*)(red + threadIdx.x * 16);
    float o = 0.f;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const float4 v = rp[q];
      o += v.x;
      o += v.y;
      o += v.z;
      o += v.w;
    }
    if (tq_bad || bad_cert) o = __builtin_nanf("");
    const size_t oi = b * 16u + threadIdx.x;
    if (a.odt == KEEP_F16) ((_Float16*)a.out)[oi] = (_Float16)o;
    else if (a.odt == KEEP_BF16) ((uint16_t*)a.out)[oi] = from_float<bf16s>(o).bits;
    else ((float*)a.out)[oi] = o;
  }
}

// ------------------------------------------------------------------ host

int64_t fl_workspace_bytes(int64_t k, int64_t I) { return FL_HDR_BYTES + k * I * 4; }

bool fl_supported(int64_t E, int64_t H, int64_t I, int64_t k, int64_t group_h, int64_t group_i) {
  if (!(H == 4096 && I % 512 == 0 && I >= 512 && I <= 2048 && k >= 1 && k <= 8 && k <= E && E <= 1024))
    return false;  // bounds first: the products below stay small
  const int64_t qtiles = k * I / 16;
  return (qtiles + FL_BLOCKS - 1) / FL_BLOCKS <= 4 && group_h >= 256 && group_h % 256 == 0 && group_i >= 256 &&
         group_i % 256 == 0 && k <= 4 * (FL_WAVES / (I / 256));
}

// All FL_BLOCKS blocks must be resident together: one block per CU.
bool fl_device_ok() {
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess) return false;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return false;
  return cus >= FL_BLOCKS;
}

// The nested tier's host-side arguments (keep_moe_layer1_nested).
struct FLNest {
  const int32_t* hot;
  int32_t nhot;
  const uint8_t *gc, *uc, *dc;
  const void *gs, *us, *ds;
  int sdt;
  int64_t group_h, group_i;
  const uint32_t* t8;
};

// The (tiles per block, slices, routes per down wave) of each served (I, k):
// gate/up q-tiles per block ceil(k I / 16 / 256), down route groups
// RG = 16 / (I / 256) of ceil(k / RG) routes.
template <int PER, bool G1, bool RES>
static bool fl_dispatch(const FLHead& h, const FLArgs& a, hipStream_t s) {
  const dim3 grid(FL_BLOCKS), blk(1024);
#define FL_K(NT, NSL, RPW)                                                                                 \
  hipLaunchKernelGGL((k_moe_layer1<NT, PER, NSL, RPW, G1, RES>), grid, blk, 0, s, h.logits, h.bias_s, h.bias_d, \
                     h.tq, h.x, h.hdr, h.E, a)
  const int k = a.k;
  switch (a.I) {
    case 2048:
      if (k <= 2) FL_K(2, 8, 1);
      else if (k <= 4) FL_K(4, 8, 2);
      else if (k <= 6) FL_K(6, 8, 3);
      else FL_K(8, 8, 4);
      return true;
    case 1536:
      if (k <= 2) FL_K(2, 6, 1);
      else if (k <= 4) FL_K(4, 6, 2);
      else if (k == 5) FL_K(4, 6, 3);
      else if (k == 6) FL_K(6, 6, 3);
      else FL_K(6, 6, 4);
      return true;
    case 1024:
      if (k <= 4) FL_K(2, 4, 1);
      else FL_K(4, 4, 2);
      return true;
    case 512:
      FL_K(2, 2, 1);
      return true;
    default:
      return false;
  }
#undef FL_K
}

void fl_launch(const float* logits, const float* bias_s, const float* bias_d, int func, int renorm, float route_scale,
               float tau, const int32_t* slot_map, int64_t S, int64_t E, int64_t k, const void* x, int x_dtype, int64_t I, const uint16_t* gc,
               const void* gs, const uint16_t* uc, const void* us, const uint16_t* dc, const void* ds, int sdt,
               int64_t group_h, int64_t group_i, const void* prepared, float limit, int32_t* idx, float* w,
               int32_t* want, float* want_score, uint8_t* admit, void* workspace, uint32_t spin_ticks, void* out,
               int odt, hipStream_t s, const FLNest* nest) {
  FLHead h{};
  h.logits = logits; h.bias_s = bias_s; h.bias_d = bias_d; h.E = (int32_t)E;
  h.x = x; h.tq = (const uint2*)((const char*)prepared + TQ_OFFSET); h.hdr = (uint32_t*)workspace;
  FLArgs a{};
  a.func = func; a.renorm = renorm;
  a.same_bias = bias_s == bias_d; a.route_scale = route_scale; a.tau = tau; a.k = (int32_t)k;
  a.slot_map = slot_map; a.S = (int32_t)(slot_map ? S : E);
  a.idx_out = idx; a.w_out = w; a.want_out = want; a.want_score_out = want_score; a.admit_out = admit;
  a.I = (int32_t)I; a.gc = gc; a.uc = uc; a.dc = dc; a.gs = gs; a.us = us; a.ds = ds; a.sdt = sdt;
  a.Gh = (int32_t)(4096 / group_h); a.gsz_h = (int32_t)group_h;
  a.Gi = (int32_t)(I / group_i); a.gsz_i = (int32_t)group_i;
  a.tq_bad = (const uint32_t*)((const char*)prepared + TQ_FLAG_OFFSET);
  a.limit = limit;
  a.qtiles = (int32_t)(k * I / 16);
  a.hx = (uint64_t*)((char*)workspace + FL_HDR_BYTES);
  a.spin_ticks = spin_ticks;
  a.out = out; a.odt = odt;
  a.xbf = x_dtype == KEEP_BF16;
  if (nest) {  // per-row fold when base and residual scales are both per row, else every slice scaled in place
    a.hot = nest->hot; a.nhot = nest->nhot;
    a.rgc = nest->gc; a.ruc = nest->uc; a.rdc = nest->dc;
    a.rgs = nest->gs; a.rus = nest->us; a.rds = nest->ds; a.rsdt = nest->sdt;
    a.rGh = (int32_t)(4096 / nest->group_h); a.rgsz_h = (int32_t)nest->group_h;
    a.rGi = (int32_t)(I / nest->group_i); a.rgsz_i = (int32_t)nest->group_i;
    a.t8 = nest->t8;
    if (group_h == 4096 && nest->group_h == 4096) {  // per-row base and residual scales: the fold
      if (E <= 384) fl_dispatch<6, true, true>(h, a, s);
      else fl_dispatch<16, true, true>(h, a, s);
    } else {
      if (E <= 384) fl_dispatch<6, false, true>(h, a, s);
      else fl_dispatch<16, false, true>(h, a, s);
    }
    return;
  }
  const bool g1 = group_h == 4096;
  if (g1) {
    if (E <= 384) fl_dispatch<6, true, false>(h, a, s);
    else fl_dispatch<16, true, false>(h, a, s);
  } else {
    if (E <= 384) fl_dispatch<6, false, false>(h, a, s);
    else fl_dispatch<16, false, false>(h, a, s);
  }
}

}  // namespace keep

using namespace keep;

extern "C" int64_t keep_moe_layer1_workspace_bytes(int64_t k, int64_t I) {
  if (!::keep::dims_ok({k, I})) return -1;
  if (k < 1 || I < 1) return -1;
  return fl_workspace_bytes(k, I);
}

// the give-up budget of every later launch, in ticks of the 100 MHz real-time counter
static std::atomic<uint32_t> g_spin_ticks{FL_SPIN_TICKS_DEFAULT};

extern "C" int keep_moe_layer1_set_spin_ticks(uint32_t ticks, uint32_t* previous) {
  KEEP_REQUIRE(ticks <= FL_SPIN_TICKS_MAX, "spin budget above %u ticks (one second)", FL_SPIN_TICKS_MAX);
  const uint32_t old = g_spin_ticks.exchange(ticks);
  if (previous) *previous = old;
  return KEEP_OK;
}

extern "C" int keep_moe_layer1_status(const void* workspace, uint32_t* status, void* stream) {
  KEEP_REQUIRE(workspace && status, "null pointer argument");
  if (hipMemcpyAsync(status, (const char*)workspace + 8, 4, hipMemcpyDeviceToHost, (hipStream_t)stream) !=
      hipSuccess)
    return launch_status("keep_moe_layer1_status");
  if (hipStreamSynchronize((hipStream_t)stream) != hipSuccess) return launch_status("keep_moe_layer1_status");
  return KEEP_OK;
}

extern "C" int keep_moe_layer1(const float* logits, const float* bias_served, const float* bias_demand,
                               int score_func, int renormalize, float route_scale, float tau,
                               const int32_t* slot_map, int64_t num_slots, int64_t E, int64_t k,
                               const void* x, int x_dtype, int64_t H, int64_t I, const uint16_t* gate_codes,
                               const void* gate_scales, const uint16_t* up_codes, const void* up_scales,
                               const uint16_t* down_codes, const void* down_scales, int scale_dtype,
                               int64_t group_size_h, int64_t group_size_i, const void* prepared, float swiglu_limit,
                               int32_t* idx, float* w, int32_t* want, float* want_score, uint8_t* admit,
                               void* workspace, int64_t workspace_bytes, void* out, int out_dtype, void* stream) {
  KEEP_REQUIRE_DIMS(num_slots, E, k, H, I, group_size_h, group_size_i);
  KEEP_REQUIRE(x_dtype == KEEP_F16 || x_dtype == KEEP_BF16, "activations must be fp16 or bf16");
  KEEP_REQUIRE(dtype_ok(scale_dtype) && dtype_ok(out_dtype), "bad dtype enum");
  KEEP_REQUIRE(score_func >= 0 && score_func <= 2, "bad score_func %d", score_func);
  KEEP_REQUIRE(group_size_h > 0 && H % group_size_h == 0 && group_size_i > 0 && I % group_size_i == 0,
               "bad group sizes");
  KEEP_REQUIRE(fl_supported(E, H, I, k, group_size_h, group_size_i),
               "shape not served by the one-launch decode layer (needs H = 4096, I a multiple of 512 up to 2048, "
               "k <= 8, E <= 1024, scale groups of 256-element multiples)");
  KEEP_REQUIRE(fl_device_ok(), "the one-launch decode layer needs %d compute units", FL_BLOCKS);
  KEEP_REQUIRE(!slot_map || (num_slots >= 1 && num_slots <= 0x7fffffffLL / (I * 512)),
               "num_slots out of range");
  KEEP_REQUIRE(logits && x && gate_codes && gate_scales && up_codes && up_scales && down_codes && down_scales &&
                   prepared && idx && w && workspace && out,
               "null pointer argument");
  KEEP_REQUIRE(workspace_bytes >= fl_workspace_bytes(k, I), "workspace needs %lld bytes, got %lld",
               (long long)fl_workspace_bytes(k, I), (long long)workspace_bytes);
  KEEP_REQUIRE(aligned(x, 16) && aligned(workspace, 256) && aligned(prepared, 16),
               "x and prepared must be 16-byte aligned, the workspace 256-byte aligned");
  KEEP_REQUIRE(aligned(gate_codes, 16) && aligned(up_codes, 16) && aligned(down_codes, 16), "codes misaligned");
  fl_launch(logits, bias_served, bias_demand, score_func, renormalize, route_scale, tau, slot_map, num_slots, E, k, x,
            x_dtype, I, gate_codes, gate_scales, up_codes, up_scales, down_codes, down_scales, scale_dtype,
            group_size_h, group_size_i, prepared, swiglu_limit, idx, w, want, want_score, admit, workspace,
            g_spin_ticks.load(std::memory_order_relaxed),
            out, out_dtype, (hipStream_t)stream, nullptr);
  return launch_status("keep_moe_layer1");
}

extern "C" int keep_moe_layer1_nested(
    const float* logits, const float* bias_served, const float* bias_demand, int score_func, int renormalize,
    float route_scale, float tau, const int32_t* slot_map, int64_t num_slots, int64_t E, int64_t k, const void* x,
    int x_dtype, int64_t H, int64_t I, const uint16_t* gate_codes, const void* gate_scales, const uint16_t* up_codes,
    const void* up_scales, const uint16_t* down_codes, const void* down_scales, int scale_dtype,
    int64_t group_size_h, int64_t group_size_i, const void* prepared, float swiglu_limit, int32_t* idx, float* w,
    int32_t* want, float* want_score, uint8_t* admit, void* workspace, int64_t workspace_bytes, void* out,
    int out_dtype, const uint32_t* hot_of_slot, int64_t num_hot, const uint8_t* res_gate_codes,
    const void* res_gate_scales, const uint8_t* res_up_codes, const void* res_up_scales,
    const uint8_t* res_down_codes, const void* res_down_scales, int res_scale_dtype, int64_t res_group_size_h,
    int64_t res_group_size_i, const uint32_t* res_table, void* stream) {
  KEEP_REQUIRE_DIMS(num_slots, E, k, H, I, group_size_h, group_size_i, num_hot, res_group_size_h, res_group_size_i);
  KEEP_REQUIRE(x_dtype == KEEP_F16 || x_dtype == KEEP_BF16, "activations must be fp16 or bf16");
  KEEP_REQUIRE(dtype_ok(scale_dtype) && dtype_ok(out_dtype) && dtype_ok(res_scale_dtype), "bad dtype enum");
  KEEP_REQUIRE(score_func >= 0 && score_func <= 2, "bad score_func %d", score_func);
  KEEP_REQUIRE(group_size_h > 0 && H % group_size_h == 0 && group_size_i > 0 && I % group_size_i == 0,
               "bad group sizes");
  KEEP_REQUIRE(fl_supported(E, H, I, k, group_size_h, group_size_i),
               "shape not served by the one-launch decode layer (needs H = 4096, I a multiple of 512 up to 2048, "
               "k <= 8, E <= 1024, scale groups of 256-element multiples)");
  KEEP_REQUIRE(res_group_size_h >= 256 && H % res_group_size_h == 0 && res_group_size_h % 256 == 0 &&
                   res_group_size_i >= 256 && I % res_group_size_i == 0 && res_group_size_i % 256 == 0,
               "residual scale groups must divide H and I and be multiples of 256");
  KEEP_REQUIRE(num_hot >= 1 && num_hot * I * H < (int64_t(1) << 31), "bad residual row count %lld",
               (long long)num_hot);
  KEEP_REQUIRE(fl_device_ok(), "the one-launch decode layer needs %d compute units", FL_BLOCKS);
  // the residual rows of the pool rows are read as E entries at most (the router's lanes)
  KEEP_REQUIRE(!slot_map || (num_slots >= 1 && num_slots <= E), "num_slots must be in 1..E with the nested tier");
  KEEP_REQUIRE(logits && x && gate_codes && gate_scales && up_codes && up_scales && down_codes && down_scales &&
                   prepared && idx && w && workspace && out && hot_of_slot && res_gate_codes && res_gate_scales &&
                   res_up_codes && res_up_scales && res_down_codes && res_down_scales && res_table,
               "null pointer argument");
  KEEP_REQUIRE(workspace_bytes >= fl_workspace_bytes(k, I), "workspace needs %lld bytes, got %lld",
               (long long)fl_workspace_bytes(k, I), (long long)workspace_bytes);
  KEEP_REQUIRE(aligned(x, 16) && aligned(workspace, 256) && aligned(prepared, 16),
               "x and prepared must be 16-byte aligned, the workspace 256-byte aligned");
  KEEP_REQUIRE(aligned(gate_codes, 16) && aligned(up_codes, 16) && aligned(down_codes, 16), "codes misaligned");
  KEEP_REQUIRE(aligned(res_gate_codes, 8) && aligned(res_up_codes, 8) && aligned(res_down_codes, 8) &&
                   aligned(hot_of_slot, 4) && aligned(res_table, 4),
               "residual codes must be 8-byte aligned");
  FLNest n{};
  n.hot = (const int32_t*)hot_of_slot; n.nhot = (int32_t)num_hot;
  n.gc = res_gate_codes; n.uc = res_up_codes; n.dc = res_down_codes;
  n.gs = res_gate_scales; n.us = res_up_scales; n.ds = res_down_scales; n.sdt = res_scale_dtype;
  n.group_h = res_group_size_h; n.group_i = res_group_size_i; n.t8 = res_table;
  fl_launch(logits, bias_served, bias_demand, score_func, renormalize, route_scale, tau, slot_map, num_slots, E, k, x,
            x_dtype, I, gate_codes, gate_scales, up_codes, up_scales, down_codes, down_scales, scale_dtype,
            group_size_h, group_size_i, prepared, swiglu_limit, idx, w, want, want_score, admit, workspace,
            g_spin_ticks.load(std::memory_order_relaxed), out, out_dtype, (hipStream_t)stream, &n);
  return launch_status("keep_moe_layer1_nested");
}
