#pragma once
// Device route plan: stable counting sort of routes by expert plus tile
// descriptors, in one workgroup of 1024 threads (no host sync, no device
// allocation): plan_block runs it in any such workgroup (k_route_plan, and the
// few-token layer's prologue with the routes held in LDS). Routes with an expert outside [0, E) sort after every valid
// route; their tiles follow the valid ones with tile_expert -1, so a GEMM
// over every descriptor writes their rows (as NaN) instead of leaving them
// unset. n_tiles_out counts the valid tiles only. With B <= E + 1 non-empty
// buckets the descriptors fit in ceil(R / tile) + E entries, since
// ceil(a / t) + ceil(b / t) <= ceil((a + b) / t) + 1.
//
// Stability: wave w owns the contiguous route range [w P, (w + 1) P), P =
// max(64, ceil(R / 16)). A route's position is its bucket's base + the routes of that
// bucket in earlier waves' ranges (per-wave histograms, scanned once) + the
// earlier routes of its own range with the same bucket: each wave walks its
// range 64 routes at a time, ranking a route among the same-bucket lanes below
// it (ballots over the bucket bits) and advancing its per-bucket offset from
// the last such lane, with no block barrier.
#include "common.h"

namespace keep {

constexpr int PLAN_THREADS = 1024;
constexpr int PLAN_WAVES = PLAN_THREADS / 64;
constexpr int PLAN_MAX_E = 1024;
constexpr int PLAN_PER = 16;  // routes per lane held in registers (R <= 16 x 64 x 16 = 16384)

// The plan's LDS scratch (78 KiB).
struct PlanLds {
  int cnt[PLAN_MAX_E + 1];
  int run[PLAN_MAX_E + 1];
  int tbase[PLAN_MAX_E + 1];
  int wh[PLAN_WAVES][PLAN_MAX_E + 1];
  int wtot[2][PLAN_WAVES];
};

// route(r): the expert of route r (any value outside [0, E) is invalid). Every
// thread of a 1024-thread workgroup calls it (it holds block barriers).
template <typename Route>
__device__ __forceinline__ void plan_block(Route route, int R, int E, int tile, int32_t* order, int32_t* inverse,
                                           int32_t* counts, int32_t* offsets, int32_t* te, int32_t* to, int32_t* tc,
                                           int max_tiles, int32_t* n_tiles_out, PlanLds& L) {
  int* cnt = L.cnt;
  int* run = L.run;
  int* tbase = L.tbase;
  int (*wh)[PLAN_MAX_E + 1] = L.wh;
  int (*wtot)[PLAN_WAVES] = L.wtot;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int EB = E + 1;  // bucket E collects invalid expert ids
  // at least 64 routes per wave, so that few routes occupy few waves
  const int P = max(64, (R + PLAN_WAVES - 1) / PLAN_WAVES);
  const int nwp = min(PLAN_WAVES, (R + P - 1) / P);     // waves holding routes
  const int r0 = min(R, wv * P), r1 = min(R, r0 + P);  // this wave's routes
  auto bucket = [&](int r) {
    const int e = route(r);
    return (e < 0 || e >= E) ? E : e;
  };
  for (int i = tid; i < nwp * EB; i += PLAN_THREADS) wh[i / EB][i % EB] = 0;
  __syncthreads();
  // up to PLAN_PER routes per lane stay in registers from here to the scatter
  const bool held = P <= 64 * PLAN_PER;
  int ev[PLAN_PER];
  if (held) {
#pragma unroll
    for (int i = 0; i < PLAN_PER; ++i) {
      const int r = r0 + i * 64 + lane;
      ev[i] = r < r1 ? bucket(r) : -1;
    }
#pragma unroll
    for (int i = 0; i < PLAN_PER; ++i)
      if (ev[i] >= 0) atomicAdd(&wh[wv][ev[i]], 1);
  } else {
    for (int r = r0 + lane; r < r1; r += 64) atomicAdd(&wh[wv][bucket(r)], 1);
  }
  __syncthreads();
  for (int e = tid; e < EB; e += PLAN_THREADS) {
    int c = 0;
    for (int w = 0; w < nwp; ++w) c += wh[w][e];
    cnt[e] = c;
  }
  __syncthreads();
  // Exclusive prefix sums of the bucket sizes (route bases) and of the tile
  // counts (first tile of each expert): buckets 2 tid, 2 tid + 1 per thread,
  // a shuffle scan inside each wave, then the 16 wave totals.
  {
    const int b0 = 2 * tid, b1 = 2 * tid + 1;
    const int c0 = b0 < EB ? cnt[b0] : 0, c1 = b1 < EB ? cnt[b1] : 0;
    const int t0 = b0 < E ? (c0 + tile - 1) / tile : 0, t1 = b1 < E ? (c1 + tile - 1) / tile : 0;
    int vc = c0 + c1, vt = t0 + t1;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const int oc = __shfl_up(vc, d, 64), ot = __shfl_up(vt, d, 64);
      if (lane >= d) {
        vc += oc;
        vt += ot;
      }
    }
    if (lane == 63) {
      wtot[0][wv] = vc;
      wtot[1][wv] = vt;
    }
    __syncthreads();
    int bc = 0, bt = 0;  // the earlier waves' totals (read together, added in wave order)
#pragma unroll
    for (int w = 0; w < PLAN_WAVES; ++w) {
      const int c = wtot[0][w], t = wtot[1][w];
      if (w < wv) {
        bc += c;
        bt += t;
      }
    }
    const int ec = bc + vc - (c0 + c1), et = bt + vt - (t0 + t1);  // exclusive
    if (b0 < EB) {
      run[b0] = ec;
      tbase[b0] = et;
    }
    if (b1 < EB) {
      run[b1] = ec + c0;
      tbase[b1] = et + t0;
    }
    if (b0 == E) n_tiles_out[0] = et;
    if (b1 == E) n_tiles_out[0] = et + t0;
  }
  __syncthreads();
  // each wave's first position in every bucket: the bucket's base plus the
  // bucket's routes in earlier waves' ranges
  for (int e = tid; e < EB; e += PLAN_THREADS) {
    int acc = run[e];
    for (int w = 0; w < nwp; ++w) {
      const int c = wh[w][e];
      wh[w][e] = acc;
      acc += c;
    }
  }
  for (int e = tid; e < E; e += PLAN_THREADS) {
    counts[e] = cnt[e];
    offsets[e] = run[e];
    const int nt = (cnt[e] + tile - 1) / tile;
    for (int i = 0; i < nt; ++i) {
      const int ti = tbase[e] + i;
      if (ti < max_tiles) {
        te[ti] = e;
        to[ti] = run[e] + i * tile;
        tc[ti] = min(tile, cnt[e] - i * tile);
      }
    }
  }
  {
    const int nbad = (cnt[E] + tile - 1) / tile;  // the invalid routes' tiles, expert -1
    for (int ti = tbase[E] + tid; ti < max_tiles; ti += PLAN_THREADS) {
      const int i = ti - tbase[E];
      const bool b = i < nbad;
      te[ti] = b ? -1 : 0;
      to[ti] = b ? run[E] + i * tile : 0;
      tc[ti] = b ? min(tile, cnt[E] - i * tile) : 0;
    }
  }
  __syncthreads();
  // stable scatter, each wave over its own range (no block barrier): a route's
  // rank among the same-bucket lanes below it, then the last of those lanes
  // advances the wave's offset for the bucket (one wave's LDS operations run in
  // order, and the offset write depends on the read before it)
  const int nbits = 32 - __builtin_clz((unsigned)E);  // bucket ids 0..E
  auto scatter = [&](int rb, int e) {  // routes rb + lane (e = -1: none)
    const int r = rb + lane;
    uint64_t peers = __ballot(e >= 0);
    for (int b = 0; b < nbits; ++b) {
      const bool bit = (e >> b) & 1;
      const uint64_t m = __ballot(bit);
      peers &= bit ? m : ~m;
    }
    if (e >= 0) {
      const int rank = __popcll(peers & ((1ull << lane) - 1ull));
      const int pos = wh[wv][e] + rank;
      const uint64_t above = lane == 63 ? 0ull : (peers >> (lane + 1));
      if (above == 0ull) wh[wv][e] = pos + 1;
      order[pos] = r;
      inverse[r] = pos;
    }
  };
  if (held) {
#pragma unroll
    for (int i = 0; i < PLAN_PER; ++i) {
      if (r0 + i * 64 >= r1) break;
      scatter(r0 + i * 64, ev[i]);
    }
  } else {
    for (int rb = r0; rb < r1; rb += 64) scatter(rb, rb + lane < r1 ? bucket(rb + lane) : -1);
  }
}

}  // namespace keep
