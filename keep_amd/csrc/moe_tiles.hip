// Routed SwiGLU MoE for a few tokens (speculative verify, T <= 256) on the
// int8 matrix cores, with the routes of one expert sharing every code load.
//
// Routes are grouped per expert by the device route plan (keep_route_plan,
// tiles of <= 16 routes of one expert), as gather_vqmm_verify_rows groups
// them (src/ramp/ops/vq_switch.py:186-225,286-377): a tile's code rows are
// read and decoded once and multiply every route of the tile, so a layer
// reads each hit expert once however many tokens hit it.
//
// Launches (no host sync, graph-capturable, all scratch in the caller's
// workspace):
//  1. k_q8_xterms: every token's int8 activation terms per 256-wide K slice
//     (three terms under a per-slice power of two, as the one-token layer
//     builds them) and the slice scales;
//  2. keep_route_plan: stable sort of the routes by expert, tile descriptors;
//  3. k_moeq_gateup_tiles: persistent, one block per CU. A unit is one tile x
//     16 rows of gate and up; 16 waves each own a K slice. Each code load is
//     decoded once (LDS image lookups) and then multiplied, with one MFMA
//     group per route, by the A operand of that route's token (rows 0-2 =
//     its three terms, DMA'd into LDS when the block enters a tile). The next
//     two units' codes are in flight while one is decoded.
//     SwiGLU in fp32, h in bf16 at its route's row;
//  4. k_moeq_down_tiles: persistent. A unit is one tile x 64 rows of down; a
//     wave owns a 256-wide K slice of h; the A operand holds two int8 terms
//     of up to 8 routes (rows 2r, 2r + 1), built once per tile. Output
//     y[route][row] in fp32;
//  5. k_moe_combine: out[t] = sum over the token's routes, in route order,
//     of w * y (a zero weight contributes nothing; an out-of-range expert
//     with a nonzero weight gives NaN), as the one-token layer combines.
//
// From the router logits (keep_moe_tiles_layer) with at most 128 routes and
// 512 experts, launches 1 and 2 and the router fold into launch 3: every
// gate/up block finds every token's served routes and plans them in LDS
// (block t also writes token t's router outputs; blocks 0 and the last one
// write the plan for launches 4 and 5), and each wave forms its K slice's x
// terms for the tile it enters. Up to 32 tokens otherwise, one prologue
// launch routes, plans and builds the terms; beyond, the router runs on its
// own launch.
#include "common.h"
#include "moe_dev.h"
#include "plan_dev.h"
#include "q8_dev.h"
#include "route_dev.h"

namespace keep {

constexpr int MT_TILE = 4;  // routes per tile: one MFMA chain serves them all in either kernel

struct MTArgs {
  const uint4* xt;     // [T][S][3][16] 16-byte slots of int8 terms
  const float* xinv;   // [T][S] 1 / (4 s)
  const int32_t *order, *te, *to, *tc, *ntiles;
  int32_t k, E, H, I, S;
  const uint16_t *gc, *uc, *dc;
  const void *gs, *us, *ds;
  int sdt;
  int32_t Gh, gsz_h, Gi, gsz_i;
  const uint4* tq;
  const uint32_t* tq_bad;
  float limit;
  uint16_t* h;  // [R, I] bf16
  float* y;     // [R, H] fp32
};

// ------------------------------------------------------------------ x terms

// Token t, K slice s (one wave): the three int8 terms of x[t] * s_slice over
// the slice's 256 values in the A-slot layout of q8_aword, and 1 / (4 s_slice).
template <bool XBF>
__device__ __forceinline__ void mt_xterms(const void* x, int H, uint4* xt, float* xinv, int t, int s, int lane) {
  const int S = H >> 8;
  const uint4 c = ldg16_q((const uint4*)x + ((size_t)t * H >> 3) + s * 32 + (lane >> 1));
  float v[4];
  q8_half4<XBF>(c, lane & 1, v);
  const float mx = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
  float sc, inv4s;
  q8_scale(rt_wave_reduce(mx, true), sc, inv4s);
  uint32_t tw[3];
  q8_terms<3>(v, sc, tw);
  uint32_t* base = (uint32_t*)(xt + ((size_t)t * S + s) * 3 * 16);
#pragma unroll
  for (int n = 0; n < 3; ++n) base[q8_aword((uint32_t)n, lane >> 1, lane & 1)] = tw[n];
  if (lane == 0) xinv[(size_t)t * S + s] = inv4s;
}

// Block t, wave s: token t's terms of slice s.
template <bool XBF>
__global__ __launch_bounds__(1024) void k_q8_xterms(const void* x, int H, uint4* xt, float* xinv) {
  mt_xterms<XBF>(x, H, xt, xinv, (int)blockIdx.x, (int)(threadIdx.x >> 6), (int)(threadIdx.x & 63));
}

// ------------------------------------------------------------------ fused prologue (few tokens)

constexpr int MT_FUSED_MAX_T = 32;  // tokens the one-block router of the prologue takes

struct MTPro {
  const void* x;
  int H;
  uint4* xt;
  float* xinv;
  const float* logits;
  const float *bias_s, *bias_d;
  int func, renorm;
  float route_scale, tau;
  const int32_t* slot_map;
  int T, E, S, k;  // S: pool rows (the plan's buckets)
  int32_t* idx;
  float* w;
  int32_t* want;
  float* want_score;
  uint8_t* admit;
  int32_t *order, *inverse, *counts, *offsets, *te, *to, *tc, *nt;
  int max_tiles;
};

// One launch in place of the router, the x terms and the route plan: block
// t < T builds token t's x terms (as k_q8_xterms); block T routes every token
// (wave w takes tokens w, w + 16, ..., each as k_router does, with the same
// outputs) and keeps the served slots in LDS, from which it runs the route
// plan (as k_route_plan over idx: plan_small up to 128 routes, else
// plan_block).
template <int PER, bool XBF>
__global__ __launch_bounds__(1024) void k_mt_prologue(MTPro p) {
  __shared__ PlanLds L;
  __shared__ int32_t s_r[MT_FUSED_MAX_T * 16];
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  if ((int)blockIdx.x < p.T) {
    if (wv < (p.H >> 8)) mt_xterms<XBF>(p.x, p.H, p.xt, p.xinv, (int)blockIdx.x, wv, lane);
    return;
  }
  for (int t = wv; t < p.T; t += 16) {
    float z[PER], bs[PER], bd[PER];
    rt_load<PER>(p.logits + (int64_t)t * p.E, p.bias_s, p.bias_d, p.E, lane, z, bs, bd);
    const RouteLane r = rt_route<PER>(z, bs, bd, p.E, p.k, p.func, p.renorm, p.route_scale, p.tau,
                                      p.bias_d == p.bias_s, lane);
    int slot = r.expert;
    if (p.slot_map) {
      int sm[PER];
      rt_load_slots<PER>(p.slot_map, p.E, lane, sm);
      slot = rt_slot_of<PER>(sm, r.valid ? r.expert : -1, p.E, p.S);
    }
    if (lane < p.k) s_r[t * p.k + lane] = r.valid ? slot : -1;
    if (r.valid) {
      const int64_t o = (int64_t)t * p.k + (lane < 32 ? lane : lane - 32);
      if (lane < 32) {
        p.idx[o] = slot;
        p.w[o] = r.value;
      } else {
        if (p.want) p.want[o] = r.expert;
        if (p.want_score) p.want_score[o] = r.value;
        if (p.admit) p.admit[o] = r.admit;
      }
    }
  }
  __syncthreads();
  auto route = [&](int r) { return s_r[r]; };
  if (p.T * p.k <= PLAN_SMALL_R)
    plan_small(route, p.T * p.k, p.S, MT_TILE, p.order, p.inverse, p.counts, p.offsets, p.te, p.to, p.tc,
               p.max_tiles, p.nt, L);
  else
    plan_block(route, p.T * p.k, p.S, MT_TILE, p.order, p.inverse, p.counts, p.offsets, p.te, p.to, p.tc,
               p.max_tiles, p.nt, L);
}

// ------------------------------------------------------------------ gate/up

// ------------------------------------------------------------------ routed gate/up (few routes)

// The routing inputs and outputs of a layer whose gate/up kernel routes its
// tokens itself (k_moeq_gateup_tiles with RPER > 0, up to PLAN_SMALL_R
// routes): every block finds every token's served routes and plans them in
// LDS. A token's served routes alone are found by rt_served_winners (no
// scores or weights where the logits certify the order); block t < T routes
// token t as k_router does and writes its router outputs, block 0 writes the
// plan's order and tiles and the last block its per-expert counts and
// offsets, for the down kernel and the combine.
struct MTRoute {
  const void* x;  // [T, H] fp16 / bf16
  const float* logits;
  const float *bias_s, *bias_d;
  int func, renorm;
  float route_scale, tau;
  const int32_t* slot_map;
  int T, E;  // tokens, router experts (the plan's buckets are the pool rows, MTArgs::E)
  int32_t* idx;
  float* w;
  int32_t* want;
  float* want_score;
  uint8_t* admit;
  int32_t *order, *inverse, *counts, *offsets, *te, *to, *tc, *nt;
  int max_tiles;
};

// The routed kernel's LDS: the served slots, the block's copy of the plan,
// and per wave the three x terms of its K slice for the current tile's four
// routes (the A-term layout of the workspace's x terms) with their 1 / (4 s).
// The unrouted kernel holds a one-entry stand-in.
template <bool ON>
struct MTRouteLds {
  static constexpr int R = ON ? PLAN_SMALL_R : 1;
  static constexpr int W = ON ? 16 : 1;
  int32_t sr[R], sb[R], order[R], te[R], to[R], tc[R];
  int32_t ntot[2];
  uint4 xl[W][MT_TILE][ON ? 48 : 1];
  float xinv[W][MT_TILE];
};

// Every wave takes tokens wv, wv + 16, ... (the served routes alone, but
// token t fully, with its router outputs, in block t); then wave 0 plans the
// block's copy (plan_small_to, with the workspace's parts as above). Every
// thread of the block calls it.
template <int PER, typename RLds>
__device__ __forceinline__ void mt_route_and_plan(const MTArgs& a, const MTRoute& p, RLds& RL) {
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  for (int t = wv; t < p.T; t += 16) {
    const bool first = t == (int)blockIdx.x;
    float z[PER], bs[PER], bd[PER];
    rt_load<PER>(p.logits + (int64_t)t * p.E, p.bias_s, p.bias_d, p.E, lane, z, bs, bd);
    int sm[PER];
    if (p.slot_map) rt_load_slots<PER>(p.slot_map, p.E, lane, sm);
    int e = -1;  // lane j < k: served route j's expert
    RouteLane r{};
    if (first) {
      r = rt_route<PER>(z, bs, bd, p.E, a.k, p.func, p.renorm, p.route_scale, p.tau, p.bias_d == p.bias_s, lane);
      e = r.valid ? r.expert : -1;
    } else {
      e = rt_served_winners<PER>(z, bs, p.E, a.k, p.func, lane);
    }
    int slot = e >= 0 && e < p.E ? e : -1;
    if (p.slot_map) slot = rt_slot_of<PER>(sm, slot, p.E, a.E);
    if (lane < a.k) RL.sr[t * a.k + lane] = slot;
    if (first && r.valid) {
      const int64_t o = (int64_t)t * a.k + (lane < 32 ? lane : lane - 32);
      if (lane < 32) {
        p.idx[o] = slot;
        p.w[o] = r.value;
      } else {
        if (p.want) p.want[o] = r.expert;
        if (p.want_score) p.want_score[o] = r.value;
        if (p.admit) p.admit[o] = r.admit;
      }
    }
  }
  rt_lds_barrier();  // the routes in LDS (the router outputs are for later launches: not waited for)
  const bool b0 = blockIdx.x == 0, bl = blockIdx.x == gridDim.x - 1;
  const PlanSmallOut o{b0 ? p.order : nullptr, b0 ? p.inverse : nullptr, bl ? p.counts : nullptr,
                       bl ? p.offsets : nullptr, b0 ? p.te : nullptr, b0 ? p.to : nullptr,
                       b0 ? p.tc : nullptr, b0 ? p.nt : nullptr, p.max_tiles, RL.order, RL.te, RL.to, RL.tc};
  plan_small_to([&](int r) { return RL.sr[r]; }, p.T * a.k, a.E, MT_TILE, o, RL.sb, RL.ntot);
}

// The two persistent kernels share one schedule. Tiles hold at most
// MT_TILE routes, so every unit of every tile is one pass over its codes and
// costs about the same: an even split of the units balances the blocks (an
// even count per block). A block's units form segments (the units of one
// tile, at most SEG of them), and run as one pipeline across them: the next
// two units' codes and scale words are in flight while one is decoded, in
// pairs over two register buffers, and those loads cross into the next
// segment, and the next tile, before the current one ends; tile and SEG
// bounds are even, so only a block's last segment can end on an odd unit.
// Loads past the block's last unit read that unit again. Wave 0 reads the
// descriptors of every tile the block touches (expert row, routes) into an
// LDS table when the kernel starts, and every wave reads its first tile
// itself, all with vector loads: a scalar load in flight would make each LDS
// wait of the decode wait for it as well. The first units' codes are issued
// after the block's small loads; a switch to a new segment waits only for
// that segment's A operands. Outputs are staged in LDS
// and written when their segment ends. The cross-wave partial sums are
// double-buffered by unit parity: a wave writes a unit's partials only after
// the barrier that the previous reader of that buffer has passed.

// A tile's first code row (expert x rows per expert), route count and routes
// (order[off + min(i, nr - 1)]).
struct MTTile {
  uint32_t row;
  int nr;
  int r[MT_TILE];
};

// Tiles a block touches, at most: ceil(units per block / units per tile) + 1,
// at most 10 for the shapes the kernels serve (checked on the host).
constexpr int MT_TPB = 16;

// Route i of the tile whose routes lanes 0-3 hold (lane i: route i), for a
// lane-dependent i: a cross-lane read, no memory. A tile's routes are never
// held in an array indexed by a lane value: the compiler would keep such an
// array per thread in LDS.
__device__ __forceinline__ int mt_route_of_lanes(int rr, uint32_t i) {
  return __builtin_amdgcn_ds_bpermute((int)(i << 2), rr);
}

// Gate/up: a unit is 16 rows of gate and of up (two code loads per wave, 32
// KiB per block). One MFMA chain per projection serves all the tile's
// routes: A row 4i + t is term t of route i's token (t < 3; row 4i + 3 is
// zero), so D rows 4i .. 4i + 2 of column j, in lane 16 i + j, are route i's
// three partial dots with weight row j.
template <bool XBF, int RPER>
__global__ __launch_bounds__(1024) void k_moeq_gateup_tiles(MTArgs a, MTRoute p) {
  constexpr int SEG = 128;  // units per segment (h staging capacity)
  constexpr bool ROUTE = RPER > 0;
  __shared__ uint4 tqs[TQR_BYTES / 16];
  __shared__ float gred[2][16][2][MT_TILE][16];  // [parity][wave][gate, up][route][row]
  __shared__ uint16_t hst[MT_TILE][SEG * 16];    // the segment's h rows
  __shared__ MTTile s_td[MT_TPB];                // the block's tiles
  __shared__ MTRouteLds<ROUTE> RL;
  const char* tq = (const char*)tqs;
  const uint32_t tq_bad = ((const __attribute__((address_space(4))) uint32_t*)a.tq_bad)[0];
  const Q8Keys lk = q8_keys(threadIdx.x & 63);
  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t j = lane & 15, g = lane >> 4;
  const bool dec = wv < a.S;  // this wave owns a K slice
  const int sl = dec ? wv : 0;
  const int rg_n = a.I >> 4;  // units per tile (>= 16)
  int nt_ = 0;
  if constexpr (!ROUTE) nt_ = __builtin_amdgcn_readfirstlane(*a.ntiles);
  // routed: the image DMA after the routing (a DMA in flight makes every wait of the routing wait for it)
  if constexpr (ROUTE) {
    mt_route_and_plan<RPER>(a, p, RL);
    nt_ = __builtin_amdgcn_readfirstlane(RL.ntot[1]);
  }
#pragma unroll
  for (int u = 0; u < 4; ++u) dma16_q(a.tq + (wv * 4 + u) * 64 + lane, tqs + (wv * 4 + u) * 64);
  const int nt = nt_;
  const int U = nt * rg_n;
  const int per = ((U + (int)gridDim.x - 1) / (int)gridDim.x + 1) & ~1;  // even: see the unit loop
  const int u0 = (int)blockIdx.x * per, u1 = min(U, u0 + per);
  if (u0 >= u1) {
    wait_vm_q<0>();
    return;
  }
  const uint32_t C = (uint32_t)a.H >> 3;
  const uint32_t kc0 = (uint32_t)sl * 32 + g * 8;
  const uint32_t grp = (uint32_t)(sl * 256) / (uint32_t)a.gsz_h;
  const uint32_t sbytes = a.sdt == KEEP_F32 ? 4u : 2u;
  struct Buf {
    uint4 q[2];
    uint32_t s[2];
  };
  const int tic0 = u0 / rg_n, ntb = (u1 - 1) / rg_n - tic0 + 1;  // the block's tiles (<= MT_TPB)
  int tic = tic0;
  // the first tile (every wave) and the next tile's row; wave 0, lane l < ntb: tile tic0 + l for the table
  int zv = 0;
  asm volatile("" : "+v"(zv));  // a lane value: these loads go through the vector unit
  // the plan's descriptors and sorted routes: the workspace's, or the block's own copy in LDS
  const int32_t* pte = ROUTE ? RL.te : a.te;
  const int32_t* pto = ROUTE ? RL.to : a.to;
  const int32_t* ptc = ROUTE ? RL.tc : a.tc;
  const int32_t* pord = ROUTE ? RL.order : a.order;
  const int te0 = pte[tic0 + zv], te1 = pte[min(tic0 + 1, nt - 1) + zv];
  const int off0 = pto[tic0 + zv], nr0 = ptc[tic0 + zv];
  const bool tl = wv == 0 && lane < ntb;
  int tte = 0, tto = 0, ttc = 1;
  if (tl) {
    tte = pte[tic0 + lane];
    tto = pto[tic0 + lane];
    ttc = ptc[tic0 + lane];
  }
  // the current and the next tile: first row and route count in scalar registers, routes from the table
  uint32_t cur_row = (uint32_t)__builtin_amdgcn_readfirstlane(te0) * (uint32_t)a.I;
  uint32_t nxt_row = (uint32_t)__builtin_amdgcn_readfirstlane(te1) * (uint32_t)a.I;
  int cur_nr = __builtin_amdgcn_readfirstlane(nr0), nxt_nr = cur_nr;
  const int rr = pord[__builtin_amdgcn_readfirstlane(off0) + min((int)(lane & 3u), cur_nr - 1)];
  int tr[MT_TILE] = {0, 0, 0, 0};
  if (tl) {
#pragma unroll
    for (int i = 0; i < MT_TILE; ++i) tr[i] = pord[tto + min(i, ttc - 1)];
  }
  // the first row of unit u (past the block's end: its last unit); u is at most two units past the
  // segment, so in tile tic or tic + 1
  auto unit_row = [&](int u) -> uint32_t {
    const int uu = min(u, u1 - 1);
    const bool n = uu >= (tic + 1) * rg_n;
    return (n ? nxt_row : cur_row) + (uint32_t)(uu - (n ? tic + 1 : tic) * rg_n) * 16u;
  };
  // a unit's codes and its rows' scale words (the aligned word holding each). Per-row scales (g1): a
  // row's slice partials are summed unscaled and its scale applied once to the sum by the SwiGLU lanes
  // (wave 0's, which hold those rows' words), so the other waves load none
  const bool g1 = a.gsz_h == a.H;
  const bool ld_scale = !g1 || wv == 0;  // wave-uniform
  auto load_unit = [&](int u, Buf& b) {
    const uint32_t row = unit_row(u) + j;
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      b.q[t] = ldg16_q((t ? a.uc : a.gc) + (size_t)row * C + kc0);
      if (ld_scale) b.s[t] = ldg4_q((const char*)(t ? a.us : a.gs) + ((row * (uint32_t)a.Gh + grp) * sbytes & ~3u));
      else b.s[t] = 0u;
    }
  };
  if (tl) s_td[lane] = MTTile{(uint32_t)tte * (uint32_t)a.I, ttc, {tr[0], tr[1], tr[2], tr[3]}};
  int us = u0, ue = min(min(u1, (tic + 1) * rg_n), u0 + SEG);
  // the segment's A operands: row j = 4i + t is term t of route i (routes past nr repeat the last one;
  // their D rows are unused), and 1 / (4 s) of the token of this lane's D rows
  q8v4 A[4];
  float inv;
  uint4 araw[4];
  auto issue_a = [&](int route_a, int route_d) {  // the routes of A row j and of this lane's D rows
    const int tok_a = route_a / a.k, tok_d = route_d / a.k;
    const uint4* asrc = a.xt + ((size_t)tok_a * a.S + sl) * 48 + min(j & 3u, 2u) * 16 + g * 4;
#pragma unroll
    for (int m = 0; m < 4; ++m) araw[m] = ldg16_q(asrc + m);
    inv = a.xinv[(size_t)tok_d * a.S + sl];
  };
  // routed: the wave forms the terms of its K slice itself, for the tile's four routes (routes past its
  // count repeat the last one), from its x chunks (issue_x), into its LDS rows; then A and 1 / (4 s)
  // read back from them as issue_a reads the workspace's
  uint4 xc[MT_TILE];
  auto issue_x = [&](int r0, int r1, int r2, int r3) {
    const int rt[MT_TILE] = {r0, r1, r2, r3};
#pragma unroll
    for (int i = 0; i < MT_TILE; ++i)
      xc[i] = ldg16_q((const uint4*)p.x + ((size_t)(rt[i] / a.k) * (uint32_t)a.H >> 3) + sl * 32 + (lane >> 1));
  };
  auto build_x = [&]() {
    if constexpr (ROUTE) {
#pragma unroll
      for (int i = 0; i < MT_TILE; ++i) {
        float v[4];
        q8_half4<XBF>(xc[i], lane & 1, v);
        const float mx = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
        float sc, inv4s;
        q8_scale(rt_wave_reduce(mx, true), sc, inv4s);
        uint32_t tw[3];
        q8_terms<3>(v, sc, tw);
        uint32_t* base = (uint32_t*)RL.xl[wv][i];
#pragma unroll
        for (int n = 0; n < 3; ++n) base[q8_aword((uint32_t)n, lane >> 1, lane & 1)] = tw[n];
        if (lane == 0) RL.xinv[wv][i] = inv4s;
      }
      // the wave reads what its other lanes wrote: one wave's LDS operations run in order, and the
      // compiler must not move the reads above the writes
      asm volatile("" ::: "memory");
      __builtin_amdgcn_wave_barrier();
      asm volatile("" ::: "memory");
      const uint4* asrc = RL.xl[wv][j >> 2] + min(j & 3u, 2u) * 16 + g * 4;
#pragma unroll
      for (int m = 0; m < 4; ++m) araw[m] = asrc[m];
      inv = RL.xinv[wv][g];
    }
  };
  auto build_a = [&]() {
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      const bool z = (j & 3u) == 3u;
      A[m] = q8v4{z ? 0 : (int)araw[m].x, z ? 0 : (int)araw[m].y, z ? 0 : (int)araw[m].z, z ? 0 : (int)araw[m].w};
    }
  };
  // the segment's staged h rows to their routes' rows
  auto flush = [&]() {
    const int rows = (ue - us) * 16;
    const uint32_t row0 = (uint32_t)(us - tic * rg_n) * 16u;
    const MTTile* td = s_td + (tic - tic0);
    int x0 = threadIdx.x;
    if constexpr (ROUTE) asm volatile("" : "+v"(x0));  // the staging address rebuilt here (held, it is spilled)
    for (int x = x0; x < cur_nr * rows; x += 1024) {
      const int i = x / rows, r = x - i * rows;
      a.h[(size_t)td->r[i] * a.I + row0 + (uint32_t)r] = hst[i][r];
    }
  };
  // the first units' codes after the block's small loads (issued before the route and A loads, they
  // measured no faster)
  Buf b0, b1;
  if constexpr (ROUTE) {
    // the codes first (they need only the tile's row), then the x chunks of its routes; the compiler waits
    // for every load before the terms are formed (the image DMA in flight makes it count them all)
    load_unit(u0, b0);
    load_unit(u0 + 1, b1);
    issue_x(__builtin_amdgcn_readfirstlane(mt_route_of_lanes(rr, 0)), __builtin_amdgcn_readfirstlane(mt_route_of_lanes(rr, 1)),
            __builtin_amdgcn_readfirstlane(mt_route_of_lanes(rr, 2)), __builtin_amdgcn_readfirstlane(mt_route_of_lanes(rr, 3)));
    wait_vm_q<0>();
    build_x();
  } else {
    issue_a(mt_route_of_lanes(rr, j >> 2), mt_route_of_lanes(rr, g));
    load_unit(u0, b0);
    load_unit(u0 + 1, b1);
    wait_vm_q<4>();  // all but the second unit's four loads: the image, A and the first unit (loads retire in order)
  }
  build_a();
  rt_lds_barrier();  // the table image and the tile table
  if (ntb > 1) {
    nxt_row = (uint32_t)__builtin_amdgcn_readfirstlane((int)s_td[1].row);
    nxt_nr = __builtin_amdgcn_readfirstlane(s_td[1].nr);
  }
  auto unit = [&](int u, Buf& b, int par) {
    const uint32_t rowc = unit_row(u);
    q8v4 B[2][4];
#pragma unroll
    for (int t = 0; t < 2; ++t) q8_decode8(tq, lk, b.q[t], B[t]);
    float scl[2];
#pragma unroll
    for (int t = 0; t < 2; ++t) scl[t] = scale_cvt(b.s[t], a.sdt, (rowc + j) * (uint32_t)a.Gh + grp);
#pragma unroll
    for (int t = 0; t < 2; ++t) asm volatile("" : "+v"(scl[t]));  // converted before b.s is reloaded
    load_unit(u + 2, b);
    __builtin_amdgcn_sched_barrier(0);
    if (dec) {
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        q8v4 acc = {0, 0, 0, 0};
#pragma unroll
        for (int m = 0; m < 4; ++m) acc = mfma_i8(A[m], B[t][m], acc);
        const float d = ((float)acc[0] + (float)acc[1] * 0.0078125f) + (float)acc[2] * 0.00006103515625f;
        if ((int)g < cur_nr) gred[par][wv][t][g][j] = g1 ? d * inv : d * inv * scl[t];
      }
    }
    rt_lds_barrier();
    // SwiGLU: thread (route i, row jj) -> the staged h rows
    if ((int)threadIdx.x < cur_nr * 16 && u < ue) {
      // the LDS address is rebuilt here, not kept across the unit loop: held, it is spilled, and a
      // reload from scratch waits for every code load in flight
      int tid = (int)threadIdx.x;
      asm volatile("" : "+v"(tid));
      const int i = tid >> 4, jj = tid & 15;
      float gsum = 0.f, usum = 0.f;
      for (int w = 0; w < a.S; ++w) {
        gsum += gred[par][w][0][i][jj];
        usum += gred[par][w][1][i][jj];
      }
      if (g1) {  // this lane's own words: row jj of the unit
        gsum *= scl[0];
        usum *= scl[1];
      }
      float hv = silu_mul(gsum, usum, a.limit);
      if (tq_bad) hv = __builtin_nanf("");
      hst[i][(u - us) * 16 + jj] = from_float<bf16s>(hv).bits;
    }
  };
  // u0 and every tile and SEG bound are even, so a segment starts on a pair and only the block's last unit
  // can be a pair's second past the end (loaded again, nothing stored)
  for (int u = u0; u < u1; u += 2) {
    if (u == ue) {      // the next segment
      rt_lds_barrier();  // every h row of this one staged
      flush();
      us = ue;
      if (us == (tic + 1) * rg_n) {
        ++tic;
        cur_row = nxt_row;
        cur_nr = nxt_nr;
        if (tic + 1 - tic0 < ntb) {
          nxt_row = (uint32_t)__builtin_amdgcn_readfirstlane((int)s_td[tic + 1 - tic0].row);
          nxt_nr = __builtin_amdgcn_readfirstlane(s_td[tic + 1 - tic0].nr);
        }
      }
      ue = min(min(u1, (tic + 1) * rg_n), us + SEG);
      const MTTile* td = s_td + (tic - tic0);
      if constexpr (ROUTE) {
        issue_x(__builtin_amdgcn_readfirstlane(td->r[0]), __builtin_amdgcn_readfirstlane(td->r[1]),
                __builtin_amdgcn_readfirstlane(td->r[2]), __builtin_amdgcn_readfirstlane(td->r[3]));
        wait_vm_q<0>();  // nothing of the switch stays in flight: the units' waits count their own loads
        build_x();
        build_a();
      } else {
        issue_a(td->r[j >> 2], td->r[g]);
        build_a();
        wait_vm_q<0>();  // nothing of the switch stays in flight: the units' waits count their own loads
      }
    }
    unit(u, b0, 0);
    unit(u + 1, b1, 1);
  }
  rt_lds_barrier();
  flush();
  wait_vm_q<0>();
}

// Down: a unit is 64 rows (four 16-row tiles, 32 KiB of codes per block);
// K slice s (I / 256 of them) has two waves, s and s + I / 256, taking row
// tiles 0-1 and 2-3. The A operand holds two int8 terms of h for each of the
// tile's routes (rows 2r, 2r + 1; rows past them zero), built in LDS by the
// slice's first wave when the block enters a segment and read by both; route
// r's dot is D rows 2r, 2r + 1. The partial sums are kept per slice and row
// tile and summed over the slices in slice order.
__global__ __launch_bounds__(1024) void k_moeq_down_tiles(MTArgs a) {
  constexpr int RT = 4;   // row tiles per unit
  constexpr int RW = 2;   // row tiles per wave
  constexpr int SEG = 48;  // units per segment (y staging capacity)
  __shared__ uint4 tqs[TQR_BYTES / 16];
  __shared__ uint4 ash[8][2 * MT_TILE * 16];         // [slice][row * 16 + slot]
  __shared__ float s_inv[8][MT_TILE];
  __shared__ float red[2][8][RT][MT_TILE][16];       // [parity][slice][row-tile][route][row]
  __shared__ float yst[MT_TILE][SEG * 16 * RT];      // the segment's y rows
  __shared__ MTTile s_td[MT_TPB];                    // the block's tiles
  const char* tq = (const char*)tqs;
  const Q8Keys lk = q8_keys(threadIdx.x & 63);
  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t j = lane & 15, g = lane >> 4;
  const int nsl = a.I >> 8;
  const bool dec = wv < 2 * nsl;  // this wave owns half of a K slice's row tiles
  const int sl = dec ? wv % nsl : 0, hf = dec ? wv / nsl : 0;
  const int rg_n = a.H / (16 * RT);  // units per tile (>= 4)
  const int nt = __builtin_amdgcn_readfirstlane(*a.ntiles);
  const int U = nt * rg_n;
  const int per = ((U + (int)gridDim.x - 1) / (int)gridDim.x + 1) & ~1;  // even: see the unit loop
  const int u0 = (int)blockIdx.x * per, u1 = min(U, u0 + per);
#pragma unroll
  for (int u = 0; u < 4; ++u) dma16_q(a.tq + (wv * 4 + u) * 64 + lane, tqs + (wv * 4 + u) * 64);
  if (u0 >= u1) {
    wait_vm_q<0>();
    return;
  }
  const uint32_t C = (uint32_t)a.I >> 3;
  const uint32_t kc0 = (uint32_t)sl * 32 + g * 8;
  const uint32_t grp = (uint32_t)(sl * 256) / (uint32_t)a.gsz_i;
  const uint32_t sbytes = a.sdt == KEEP_F32 ? 4u : 2u;
  struct Buf {
    uint4 q[RW];
    uint32_t s[RW];
  };
  const int tic0 = u0 / rg_n, ntb = (u1 - 1) / rg_n - tic0 + 1;  // the block's tiles (<= MT_TPB)
  int tic = tic0;
  // the first tile (every wave) and the next tile's row; wave 0, lane l < ntb: tile tic0 + l for the table
  int zv = 0;
  asm volatile("" : "+v"(zv));  // a lane value: these loads go through the vector unit
  const int te0 = a.te[tic0 + zv], te1 = a.te[min(tic0 + 1, nt - 1) + zv];
  const int off0 = a.to[tic0 + zv], nr0 = a.tc[tic0 + zv];
  const bool tl = wv == 0 && lane < ntb;
  int tte = 0, tto = 0, ttc = 1;
  if (tl) {
    tte = a.te[tic0 + lane];
    tto = a.to[tic0 + lane];
    ttc = a.tc[tic0 + lane];
  }
  // the current and the next tile: first row and route count in scalar registers, routes from the table
  uint32_t cur_row = (uint32_t)__builtin_amdgcn_readfirstlane(te0) * (uint32_t)a.H;
  uint32_t nxt_row = (uint32_t)__builtin_amdgcn_readfirstlane(te1) * (uint32_t)a.H;
  int cur_nr = __builtin_amdgcn_readfirstlane(nr0), nxt_nr = cur_nr;
  const int rr = a.order[__builtin_amdgcn_readfirstlane(off0) + min((int)(lane & 3u), cur_nr - 1)];
  int tr[MT_TILE] = {0, 0, 0, 0};
  if (tl) {
#pragma unroll
    for (int i = 0; i < MT_TILE; ++i) tr[i] = a.order[tto + min(i, ttc - 1)];
  }
  // the first row of unit u (past the block's end: its last unit); u is at most two units past the
  // segment, so in tile tic or tic + 1
  auto unit_row = [&](int u) -> uint32_t {
    const int uu = min(u, u1 - 1);
    const bool n = uu >= (tic + 1) * rg_n;
    return (n ? nxt_row : cur_row) + (uint32_t)(uu - (n ? tic + 1 : tic) * rg_n) * (16u * RT);
  };
  // a unit's codes and its rows' scale words (the aligned word holding each)
  auto load_unit = [&](int u, Buf& b) {  // this wave's row tiles 2 hf, 2 hf + 1
    const uint32_t rbase = unit_row(u) + (uint32_t)hf * (16u * RW) + j;
#pragma unroll
    for (int rt = 0; rt < RW; ++rt) {
      b.q[rt] = ldg16_q(a.dc + (size_t)(rbase + (uint32_t)rt * 16u) * C + kc0);
      b.s[rt] = ldg4_q((const char*)a.ds + (((rbase + (uint32_t)rt * 16u) * (uint32_t)a.Gi + grp) * sbytes & ~3u));
    }
  };
  if (tl) s_td[lane] = MTTile{(uint32_t)tte * (uint32_t)a.H, ttc, {tr[0], tr[1], tr[2], tr[3]}};
  int us = u0, ue = min(min(u1, (tic + 1) * rg_n), u0 + SEG);
  // the segment's A operands: the slice's first wave writes the tile's h slices as two int8 terms per
  // route into the slice's LDS rows; after a block barrier both waves of the slice read their A
  // fragments and the 1 / (4 s) of their D rows
  q8v4 A[4];
  float inv[2];
  auto build_a = [&](int r0, int r1, int r2, int r3) {  // the tile's routes (past nr: the last one again)
    if (dec && hf == 0) {
      const int rt4[MT_TILE] = {r0, r1, r2, r3};
      uint4 hq[MT_TILE];
#pragma unroll
      for (int i = 0; i < MT_TILE; ++i)
        hq[i] = ldg16_q((const uint4*)(a.h + (size_t)rt4[i] * a.I) + sl * 32 + (lane >> 1));
      uint32_t* aw = (uint32_t*)ash[sl];
#pragma unroll
      for (int i = 0; i < MT_TILE; ++i) {
        float v[4];
        q8_half4<true>(hq[i], lane & 1, v);
        const float mx = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
        float sc, inv4s;
        q8_scale(rt_wave_reduce(mx, true), sc, inv4s);
        uint32_t tw[2];
        q8_digits2(v, sc, tw);
        aw[q8_aword((uint32_t)(2 * i), lane >> 1, lane & 1)] = tw[0];
        aw[q8_aword((uint32_t)(2 * i + 1), lane >> 1, lane & 1)] = tw[1];
        if (lane == 0) s_inv[sl][i] = inv4s;
      }
    }
  };
  auto read_a = [&]() {  // after the barrier that follows build_a
    if (dec) {
      // the LDS addresses are rebuilt here, not kept across the unit loop: held, one is spilled, and its
      // reload from scratch waits for every code load in flight
      uint32_t g = lane >> 4;
      asm volatile("" : "+v"(g));
      const q8v4* as = (const q8v4*)ash[sl] + (j & (2 * MT_TILE - 1)) * 16 + g * 4;
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        const q8v4 v = as[m];
        const bool z = (int)j >= 2 * cur_nr;  // rows past the tile's routes
        A[m] = q8v4{z ? 0 : v[0], z ? 0 : v[1], z ? 0 : v[2], z ? 0 : v[3]};
      }
#pragma unroll
      for (int h2 = 0; h2 < 2; ++h2) inv[h2] = s_inv[sl][min(2 * (int)g + h2, MT_TILE - 1)];
    }
  };
  // the segment's staged y rows to their routes' rows
  auto flush = [&]() {
    const int rows = (ue - us) * 16 * RT;
    const uint32_t row0 = (uint32_t)(us - tic * rg_n) * (16u * RT);
    const MTTile* td = s_td + (tic - tic0);
    for (int x = threadIdx.x; x < cur_nr * rows; x += 1024) {
      const int i = x / rows, r = x - i * rows;
      a.y[(size_t)td->r[i] * a.H + row0 + (uint32_t)r] = yst[i][r];
    }
  };
  // the first units' codes after the block's small loads (issued before the route and A loads, they
  // measured no faster)
  build_a(__builtin_amdgcn_readlane(rr, 0), __builtin_amdgcn_readlane(rr, 1), __builtin_amdgcn_readlane(rr, 2),
          __builtin_amdgcn_readlane(rr, 3));
  Buf b0, b1;
  load_unit(u0, b0);
  load_unit(u0 + 1, b1);
  wait_vm_q<2 * RW>();  // all but the second unit's loads: the image, h and the first unit (loads retire in order)
  rt_lds_barrier();  // the table image, the tile table and the A terms
  read_a();
  if (ntb > 1) {
    nxt_row = (uint32_t)__builtin_amdgcn_readfirstlane((int)s_td[1].row);
    nxt_nr = __builtin_amdgcn_readfirstlane(s_td[1].nr);
  }
  auto unit = [&](int u, Buf& b, int par) {
    const uint32_t rowc = unit_row(u);
    const uint32_t rowh = rowc + (uint32_t)hf * (16u * RW);
    q8v4 B[RW][4];
#pragma unroll
    for (int rt = 0; rt < RW; ++rt) q8_decode8(tq, lk, b.q[rt], B[rt]);
    float scl[RW];
#pragma unroll
    for (int rt = 0; rt < RW; ++rt)
      scl[rt] = scale_cvt(b.s[rt], a.sdt, (rowh + (uint32_t)rt * 16u + j) * (uint32_t)a.Gi + grp);
#pragma unroll
    for (int rt = 0; rt < RW; ++rt) asm volatile("" : "+v"(scl[rt]));  // converted before b.s is reloaded
    load_unit(u + 2, b);
    __builtin_amdgcn_sched_barrier(0);
    if (dec) {
#pragma unroll
      for (int rt = 0; rt < RW; ++rt) {
        q8v4 acc = {0, 0, 0, 0};
#pragma unroll
        for (int m = 0; m < 4; ++m) acc = mfma_i8(A[m], B[rt][m], acc);
        // route r: rows 2r, 2r + 1 = lanes 16 (r / 2) + j, registers 2 (r % 2), 2 (r % 2) + 1
#pragma unroll
        for (int h2 = 0; h2 < 2; ++h2) {
          const int r = 2 * (int)g + h2;
          if (r < cur_nr) {
            const float d = h2 ? (float)acc[2] + (float)acc[3] * 0.0078125f : (float)acc[0] + (float)acc[1] * 0.0078125f;
            red[par][sl][hf * RW + rt][r][j] = d * inv[h2] * scl[rt];
          }
        }
      }
    }
    rt_lds_barrier();
    if ((int)threadIdx.x < cur_nr * 16 * RT && u < ue) {
      const int i = threadIdx.x / (16 * RT), rt = (threadIdx.x >> 4) % RT, jj = threadIdx.x & 15;
      float v = 0.f;
      for (int w = 0; w < nsl; ++w) v += red[par][w][rt][i][jj];
      yst[i][(u - us) * 16 * RT + rt * 16 + jj] = v;
    }
  };
  // u0 and every tile and SEG bound are even, so a segment starts on a pair and only the block's last unit
  // can be a pair's second past the end (loaded again, nothing stored)
  for (int u = u0; u < u1; u += 2) {
    if (u == ue) {      // the next segment
      rt_lds_barrier();  // every y row of this one staged
      flush();
      us = ue;
      if (us == (tic + 1) * rg_n) {
        ++tic;
        cur_row = nxt_row;
        cur_nr = nxt_nr;
        if (tic + 1 - tic0 < ntb) {
          nxt_row = (uint32_t)__builtin_amdgcn_readfirstlane((int)s_td[tic + 1 - tic0].row);
          nxt_nr = __builtin_amdgcn_readfirstlane(s_td[tic + 1 - tic0].nr);
        }
      }
      ue = min(min(u1, (tic + 1) * rg_n), us + SEG);
      const MTTile* td = s_td + (tic - tic0);
      build_a(__builtin_amdgcn_readfirstlane(td->r[0]), __builtin_amdgcn_readfirstlane(td->r[1]),
              __builtin_amdgcn_readfirstlane(td->r[2]), __builtin_amdgcn_readfirstlane(td->r[3]));
      rt_lds_barrier();  // the segment's A terms
      read_a();
    }
    unit(u, b0, 0);
    unit(u + 1, b1, 1);
  }
  rt_lds_barrier();
  flush();
  wait_vm_q<0>();
}

// ------------------------------------------------------------------ combine

__global__ __launch_bounds__(256) void k_moe_combine(const float* y, const int32_t* idx, const float* w, int T,
                                                     int k, int E, int H, const uint32_t* tq_bad, void* out,
                                                     int odt) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (int64_t)T * H) return;
  const int t = (int)(i / H), n = (int)(i - (int64_t)t * H);
  // every route's expert, weight and row value in flight together (the rows
  // of y are always readable; an absent route's is simply not used): one
  // memory round trip, then the sum in route order
  constexpr int KC = 8;
  float o = 0.f;
  bool bad = false;
  for (int r0 = 0; r0 < k; r0 += KC) {
    int e[KC];
    float wt[KC], yv[KC];
#pragma unroll
    for (int r = 0; r < KC; ++r) {
      const int rr = min(r0 + r, k - 1);
      e[r] = idx[t * k + rr];
      wt[r] = w[t * k + rr];
      yv[r] = y[(int64_t)(t * k + rr) * H + n];
    }
#pragma unroll
    for (int r = 0; r < KC; ++r) {
      if (r0 + r < k) {
        const bool ok = e[r] >= 0 && e[r] < E;
        bad |= wt[r] != 0.f && !ok;
        if (ok && wt[r] != 0.f) o = fmaf(wt[r], yv[r], o);
      }
    }
  }
  if (bad || *tq_bad) o = __builtin_nanf("");
  if (odt == KEEP_F16) ((_Float16*)out)[i] = (_Float16)o;
  else if (odt == KEEP_BF16) ((uint16_t*)out)[i] = from_float<bf16s>(o).bits;
  else ((float*)out)[i] = o;
}

// ------------------------------------------------------------------ host

struct MTWorkspace {
  size_t xt, xinv, order, inverse, counts, offsets, te, to, tc, nt, y, total;
  int64_t max_tiles;
};

static size_t mt_align(size_t v) { return (v + 255) & ~(size_t)255; }

static MTWorkspace mt_layout(int64_t T, int64_t k, int64_t E, int64_t H) {
  MTWorkspace w{};
  const int64_t R = T * k, S = H / 256;
  w.max_tiles = (R + MT_TILE - 1) / MT_TILE + E;
  size_t o = 0;
  w.xt = o; o = mt_align(o + (size_t)T * S * 3 * 256);
  w.xinv = o; o = mt_align(o + (size_t)T * S * 4);
  w.order = o; o = mt_align(o + (size_t)R * 4);
  w.inverse = o; o = mt_align(o + (size_t)R * 4);
  w.counts = o; o = mt_align(o + (size_t)E * 4);
  w.offsets = o; o = mt_align(o + (size_t)E * 4);
  w.te = o; o = mt_align(o + (size_t)w.max_tiles * 4);
  w.to = o; o = mt_align(o + (size_t)w.max_tiles * 4);
  w.tc = o; o = mt_align(o + (size_t)w.max_tiles * 4);
  w.nt = o; o = mt_align(o + 4);
  w.y = o; o = mt_align(o + (size_t)R * H * 4);
  w.total = o;
  return w;
}

// Grid of a persistent expert kernel over tiles of `units` units each (mt_tail), and the most tiles one
// of its blocks can touch: its units (ceil(tiles x units / grid), rounded up to even) may start at a
// tile's last unit.
static int64_t mt_grid(int64_t tiles_ub, int64_t units) {
  return std::max<int64_t>(1, std::min<int64_t>(256, tiles_ub * units));
}
static int64_t mt_tiles_per_block(int64_t tiles_ub, int64_t units) {
  const int64_t per = ((tiles_ub * units + mt_grid(tiles_ub, units) - 1) / mt_grid(tiles_ub, units) + 1) & ~1LL;
  return (per + units - 1) / units + 1;
}

// Tiles of one layer, at most: each holds at least one route.
static int64_t mt_tiles_ub(int64_t T, int64_t k, int64_t E) {
  const int64_t R = T * k;
  return std::min<int64_t>(R, (R + MT_TILE - 1) / MT_TILE + E);
}

bool moe_tiles_supported(int64_t T, int64_t E, int64_t H, int64_t I, int64_t k, int64_t group_h, int64_t group_i) {
  return T >= 1 && T <= 256 && k >= 1 && k <= 16 && k <= E && E >= 1 && E <= 1024 && H % 256 == 0 && H <= 4096 &&
         I % 256 == 0 && I <= 2048 && group_h % 256 == 0 && group_i % 256 == 0 && (int64_t)E * I <= 0x7fffffffLL &&
         (int64_t)E * H <= 0x7fffffffLL && mt_tiles_per_block(mt_tiles_ub(T, k, E), I / 16) <= MT_TPB &&
         mt_tiles_per_block(mt_tiles_ub(T, k, E), H / 64) <= MT_TPB;
}

}  // namespace keep

using namespace keep;

// Route-plan launch (plan.hip).
extern "C" int keep_route_plan(const int32_t* rhs, int64_t R, int64_t E, int64_t tile, int32_t* order,
                               int32_t* inverse, int32_t* counts, int32_t* offsets, int32_t* tile_expert,
                               int32_t* tile_offset, int32_t* tile_count, int64_t max_tiles, int32_t* n_tiles_out,
                               void* stream);

extern "C" int64_t keep_moe_tiles_workspace_bytes(int64_t T, int64_t k, int64_t num_experts, int64_t H) {
  if (!::keep::dims_ok({T, k, num_experts, H})) return -1;
  if (T < 0 || k < 1 || num_experts < 1 || H < 256) return -1;
  return (int64_t)mt_layout(T, k, num_experts, H).total;
}

extern "C" int keep_moe_tiles_supported(int64_t T, int64_t num_experts, int64_t H, int64_t I, int64_t k,
                                        int64_t group_size_h, int64_t group_size_i) {
  if (!::keep::dims_ok({T, num_experts, H, I, k, group_size_h, group_size_i})) return 0;
  return moe_tiles_supported(T, num_experts, H, I, k, group_size_h, group_size_i) ? 1 : 0;
}

// The checks both few-token entry points make on the expert side.
static int mt_check(const void* x, int x_dtype, int64_t T, int64_t H, int64_t I, int64_t k, int64_t num_experts,
                    const uint16_t* gate_codes, const void* gate_scales, const uint16_t* up_codes,
                    const void* up_scales, const uint16_t* down_codes, const void* down_scales, int scale_dtype,
                    int64_t group_size_h, int64_t group_size_i, const void* prepared, void* h_work, void* workspace,
                    int64_t workspace_bytes, void* out, int out_dtype) {
  KEEP_REQUIRE(x_dtype == KEEP_F16 || x_dtype == KEEP_BF16, "activations must be fp16 or bf16");
  KEEP_REQUIRE(dtype_ok(scale_dtype) && dtype_ok(out_dtype), "bad dtype enum");
  KEEP_REQUIRE(group_size_h > 0 && H % group_size_h == 0 && group_size_i > 0 && I % group_size_i == 0,
               "bad group sizes");
  KEEP_REQUIRE(moe_tiles_supported(T, num_experts, H, I, k, group_size_h, group_size_i),
               "shape not served by the tiled MoE kernels (T <= 256, k <= 16, E <= 1024, H a multiple of 256 up "
               "to 4096, I a multiple of 256 up to 2048, scale groups of 256-element multiples)");
  KEEP_REQUIRE(x && gate_codes && gate_scales && up_codes && up_scales && down_codes && down_scales && prepared &&
                   h_work && workspace && out,
               "null pointer argument");
  const MTWorkspace L = mt_layout(T, k, num_experts, H);
  KEEP_REQUIRE(workspace_bytes >= (int64_t)L.total, "workspace needs %lld bytes, got %lld", (long long)L.total,
               (long long)workspace_bytes);
  KEEP_REQUIRE(aligned(x, 16) && aligned(h_work, 16) && aligned(prepared, 16) && aligned(workspace, 256),
               "x, h_work and prepared must be 16-byte aligned and the workspace 256-byte aligned");
  KEEP_REQUIRE(aligned(gate_codes, 16) && aligned(up_codes, 16) && aligned(down_codes, 16), "codes misaligned");
  return KEEP_OK;
}

static MTArgs mt_args(int64_t H, int64_t I, int64_t k, int64_t num_experts, const uint16_t* gate_codes,
                      const void* gate_scales, const uint16_t* up_codes, const void* up_scales,
                      const uint16_t* down_codes, const void* down_scales, int scale_dtype, int64_t group_size_h,
                      int64_t group_size_i, const void* prepared, float swiglu_limit, void* h_work, char* ws,
                      const MTWorkspace& L) {
  MTArgs a{};
  a.xt = (const uint4*)(ws + L.xt);
  a.xinv = (const float*)(ws + L.xinv);
  a.order = (const int32_t*)(ws + L.order);
  a.te = (const int32_t*)(ws + L.te);
  a.to = (const int32_t*)(ws + L.to);
  a.tc = (const int32_t*)(ws + L.tc);
  a.ntiles = (const int32_t*)(ws + L.nt);
  a.k = (int32_t)k; a.E = (int32_t)num_experts; a.H = (int32_t)H; a.I = (int32_t)I; a.S = (int32_t)(H / 256);
  a.gc = gate_codes; a.uc = up_codes; a.dc = down_codes; a.gs = gate_scales; a.us = up_scales; a.ds = down_scales;
  a.sdt = scale_dtype; a.Gh = (int32_t)(H / group_size_h); a.gsz_h = (int32_t)group_size_h;
  a.Gi = (int32_t)(I / group_size_i); a.gsz_i = (int32_t)group_size_i;
  a.tq = (const uint4*)((const char*)prepared + TQR_OFFSET);
  a.tq_bad = (const uint32_t*)((const char*)prepared + TQ_FLAG_OFFSET);
  a.limit = swiglu_limit;
  a.h = (uint16_t*)h_work;
  a.y = (float*)(ws + L.y);
  return a;
}

// The gate/up launch: unrouted (rp null: x terms and plan in the workspace) or routing its tokens itself
// with `per` (<= 8) logits per router lane.
template <bool XBF>
static void mt_launch_gateup(const MTArgs& a, const MTRoute* rp, int per, unsigned g1, hipStream_t s) {
  if (!rp) {
    hipLaunchKernelGGL((k_moeq_gateup_tiles<XBF, 0>), dim3(g1), dim3(1024), 0, s, a, MTRoute{});
  } else if (per <= 2) {
    hipLaunchKernelGGL((k_moeq_gateup_tiles<XBF, 2>), dim3(g1), dim3(1024), 0, s, a, *rp);
  } else if (per <= 4) {
    hipLaunchKernelGGL((k_moeq_gateup_tiles<XBF, 4>), dim3(g1), dim3(1024), 0, s, a, *rp);
  } else if (per <= 6) {
    hipLaunchKernelGGL((k_moeq_gateup_tiles<XBF, 6>), dim3(g1), dim3(1024), 0, s, a, *rp);
  } else {
    hipLaunchKernelGGL((k_moeq_gateup_tiles<XBF, 8>), dim3(g1), dim3(1024), 0, s, a, *rp);
  }
}

// gate/up, down and the combine, once the x terms and the plan are in the workspace (rp null), or with
// the gate/up kernel routing and planning (rp: its routing arguments, per: logits per router lane).
static void mt_tail(const MTArgs& a, int x_dtype, int64_t T, int64_t H, int64_t I, int64_t k, int64_t num_experts,
                    const int32_t* idx, const float* w, const MTWorkspace& L, void* out, int out_dtype,
                    hipStream_t s, const MTRoute* rp = nullptr, int per = 0) {
  const int64_t tiles_ub = mt_tiles_ub(T, k, num_experts);
  const unsigned g1 = (unsigned)mt_grid(tiles_ub, I / 16);
  const unsigned g2 = (unsigned)mt_grid(tiles_ub, H / 64);
  if (x_dtype == KEEP_BF16) mt_launch_gateup<true>(a, rp, per, g1, s);
  else mt_launch_gateup<false>(a, rp, per, g1, s);
  hipLaunchKernelGGL(k_moeq_down_tiles, dim3(g2), dim3(1024), 0, s, a);
  const int64_t n = T * H;
  hipLaunchKernelGGL(k_moe_combine, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, a.y, idx, w, (int)T, (int)k,
                     (int)num_experts, (int)H, a.tq_bad, out, out_dtype);
}

extern "C" int keep_moe_tiles(const void* x, int x_dtype, int64_t T, int64_t H, int64_t I, const int32_t* idx,
                              const float* w, int64_t k, int64_t num_experts, const uint16_t* gate_codes,
                              const void* gate_scales, const uint16_t* up_codes, const void* up_scales,
                              const uint16_t* down_codes, const void* down_scales, int scale_dtype,
                              int64_t group_size_h, int64_t group_size_i, const void* prepared, float swiglu_limit,
                              void* h_work, void* workspace, int64_t workspace_bytes, void* out, int out_dtype,
                              void* stream) {
  KEEP_REQUIRE_DIMS(T, H, I, k, num_experts, group_size_h, group_size_i);
  const int chk = mt_check(x, x_dtype, T, H, I, k, num_experts, gate_codes, gate_scales, up_codes, up_scales,
                           down_codes, down_scales, scale_dtype, group_size_h, group_size_i, prepared, h_work,
                           workspace, workspace_bytes, out, out_dtype);
  if (chk != KEEP_OK) return chk;
  KEEP_REQUIRE(idx && w, "null pointer argument");
  hipStream_t s = (hipStream_t)stream;
  char* ws = (char*)workspace;
  const MTWorkspace L = mt_layout(T, k, num_experts, H);
  const MTArgs a = mt_args(H, I, k, num_experts, gate_codes, gate_scales, up_codes, up_scales, down_codes,
                           down_scales, scale_dtype, group_size_h, group_size_i, prepared, swiglu_limit, h_work, ws, L);
  const int64_t R = T * k;
  const dim3 xb((unsigned)(64 * (H / 256)));
  if (x_dtype == KEEP_BF16)
    hipLaunchKernelGGL((k_q8_xterms<true>), dim3((unsigned)T), xb, 0, s, x, (int)H, (uint4*)(ws + L.xt),
                       (float*)(ws + L.xinv));
  else
    hipLaunchKernelGGL((k_q8_xterms<false>), dim3((unsigned)T), xb, 0, s, x, (int)H, (uint4*)(ws + L.xt),
                       (float*)(ws + L.xinv));
  const int rc = keep_route_plan(idx, R, num_experts, MT_TILE, (int32_t*)(ws + L.order), (int32_t*)(ws + L.inverse),
                                 (int32_t*)(ws + L.counts), (int32_t*)(ws + L.offsets), (int32_t*)(ws + L.te),
                                 (int32_t*)(ws + L.to), (int32_t*)(ws + L.tc), L.max_tiles, (int32_t*)(ws + L.nt),
                                 stream);
  if (rc != KEEP_OK) return rc;
  mt_tail(a, x_dtype, T, H, I, k, num_experts, idx, w, L, out, out_dtype, s);
  return launch_status("keep_moe_tiles");
}

// Router declaration (router.hip).
extern "C" int keep_router_dual_topk(const float* logits, int64_t T, int64_t E, int64_t k, const float* bias_served,
                                     const float* bias_demand, int score_func, int renormalize, float route_scale,
                                     float tau, const int32_t* slot_map, int64_t num_slots, int32_t* idx, float* w,
                                     int32_t* want, float* want_score, uint8_t* admit, void* stream);

extern "C" int keep_moe_tiles_layer(const float* logits, const float* bias_served, const float* bias_demand,
                                    int score_func, int renormalize, float route_scale, float tau,
                                    const int32_t* slot_map, int64_t num_slots, int64_t num_experts, int64_t k,
                                    const void* x, int x_dtype, int64_t T, int64_t H, int64_t I,
                                    const uint16_t* gate_codes, const void* gate_scales, const uint16_t* up_codes,
                                    const void* up_scales, const uint16_t* down_codes, const void* down_scales,
                                    int scale_dtype, int64_t group_size_h, int64_t group_size_i,
                                    const void* prepared, float swiglu_limit, int32_t* idx, float* w, int32_t* want,
                                    float* want_score, uint8_t* admit, void* h_work, void* workspace,
                                    int64_t workspace_bytes, void* out, int out_dtype, void* stream) {
  KEEP_REQUIRE_DIMS(num_slots, num_experts, k, T, H, I, group_size_h, group_size_i);
  KEEP_REQUIRE(num_experts >= 1 && num_experts <= 64 * RT_MAX_PER_LANE, "num_experts must be in 1..%d",
               64 * RT_MAX_PER_LANE);
  KEEP_REQUIRE(score_func >= 0 && score_func <= 2, "bad score_func %d", score_func);
  KEEP_REQUIRE(!slot_map || (num_slots >= 1 && num_slots <= 1024), "num_slots must be in 1..1024");
  const int64_t S = slot_map ? num_slots : num_experts;  // pool rows
  const int chk = mt_check(x, x_dtype, T, H, I, k, S, gate_codes, gate_scales, up_codes, up_scales, down_codes,
                           down_scales, scale_dtype, group_size_h, group_size_i, prepared, h_work, workspace,
                           workspace_bytes, out, out_dtype);
  if (chk != KEEP_OK) return chk;
  KEEP_REQUIRE(k <= num_experts, "k must be <= num_experts");
  KEEP_REQUIRE(logits && idx && w, "null pointer argument");
  if (T > MT_FUSED_MAX_T) {  // the router on its own launch (one wave per token), then keep_moe_tiles
    const int rc = keep_router_dual_topk(logits, T, num_experts, k, bias_served, bias_demand, score_func, renormalize,
                                         route_scale, tau, slot_map, num_slots, idx, w, want, want_score, admit,
                                         stream);
    if (rc != KEEP_OK) return rc;
    return keep_moe_tiles(x, x_dtype, T, H, I, idx, w, k, S, gate_codes, gate_scales, up_codes, up_scales,
                          down_codes, down_scales, scale_dtype, group_size_h, group_size_i, prepared, swiglu_limit,
                          h_work, workspace, workspace_bytes, out, out_dtype, stream);
  }
  hipStream_t s = (hipStream_t)stream;
  char* ws = (char*)workspace;
  const MTWorkspace L = mt_layout(T, k, S, H);
  const MTArgs a = mt_args(H, I, k, S, gate_codes, gate_scales, up_codes, up_scales, down_codes, down_scales,
                           scale_dtype, group_size_h, group_size_i, prepared, swiglu_limit, h_work, ws, L);
  const int per = (int)((num_experts + 63) / 64);
  // up to 128 routes and 512 experts the gate/up kernel routes and plans in every block (no prologue launch;
  // a router lane holding 16 logits would spill inside it); every block of it routes a token fully
  if (T * k <= PLAN_SMALL_R && per <= 8 && T <= mt_grid(mt_tiles_ub(T, k, S), I / 16)) {
    MTRoute rp{};
    rp.x = x; rp.logits = logits; rp.bias_s = bias_served; rp.bias_d = bias_demand; rp.func = score_func;
    rp.renorm = renormalize; rp.route_scale = route_scale; rp.tau = tau; rp.slot_map = slot_map;
    rp.T = (int)T; rp.E = (int)num_experts;
    rp.idx = idx; rp.w = w; rp.want = want; rp.want_score = want_score; rp.admit = admit;
    rp.order = (int32_t*)(ws + L.order); rp.inverse = (int32_t*)(ws + L.inverse);
    rp.counts = (int32_t*)(ws + L.counts); rp.offsets = (int32_t*)(ws + L.offsets); rp.te = (int32_t*)(ws + L.te);
    rp.to = (int32_t*)(ws + L.to); rp.tc = (int32_t*)(ws + L.tc); rp.nt = (int32_t*)(ws + L.nt);
    rp.max_tiles = (int)L.max_tiles;
    mt_tail(a, x_dtype, T, H, I, k, S, idx, w, L, out, out_dtype, s, &rp, per);
    return launch_status("keep_moe_tiles_layer");
  }
  MTPro p{};
  p.x = x; p.H = (int)H; p.xt = (uint4*)(ws + L.xt); p.xinv = (float*)(ws + L.xinv);
  p.logits = logits; p.bias_s = bias_served; p.bias_d = bias_demand; p.func = score_func; p.renorm = renormalize;
  p.route_scale = route_scale; p.tau = tau; p.slot_map = slot_map;
  p.T = (int)T; p.E = (int)num_experts; p.S = (int)S; p.k = (int)k;
  p.idx = idx; p.w = w; p.want = want; p.want_score = want_score; p.admit = admit;
  p.order = (int32_t*)(ws + L.order); p.inverse = (int32_t*)(ws + L.inverse); p.counts = (int32_t*)(ws + L.counts);
  p.offsets = (int32_t*)(ws + L.offsets); p.te = (int32_t*)(ws + L.te); p.to = (int32_t*)(ws + L.to);
  p.tc = (int32_t*)(ws + L.tc); p.nt = (int32_t*)(ws + L.nt); p.max_tiles = (int)L.max_tiles;
  const dim3 grid((unsigned)(T + 1)), blk(1024);
#define MT_PRO(P)                                                                        \
  do {                                                                                   \
    if (x_dtype == KEEP_BF16) hipLaunchKernelGGL((k_mt_prologue<P, true>), grid, blk, 0, s, p); \
    else hipLaunchKernelGGL((k_mt_prologue<P, false>), grid, blk, 0, s, p);             \
  } while (0)
  if (per <= 1) MT_PRO(1);
  else if (per <= 2) MT_PRO(2);
  else if (per <= 4) MT_PRO(4);
  else if (per <= 6) MT_PRO(6);
  else if (per <= 8) MT_PRO(8);
  else MT_PRO(16);
#undef MT_PRO
  mt_tail(a, x_dtype, T, H, I, k, S, idx, w, L, out, out_dtype, s);
  return launch_status("keep_moe_tiles_layer");
}
