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

constexpr int PLAN_SMALL_R = 128;  // routes plan_small takes: two per lane of one wave

// Where plan_small_to writes. Every global pointer may be null (not written);
// l_order / l_te / l_to / l_tc, when not null, receive LDS copies of order and
// of the tile descriptors (at most R tiles).
struct PlanSmallOut {
  int32_t *order, *inverse, *counts, *offsets, *te, *to, *tc, *n_tiles;
  int max_tiles;
  int32_t *l_order, *l_te, *l_to, *l_tc;
};

// plan_block's outputs for R <= PLAN_SMALL_R, with one block barrier. Wave 0
// holds routes lane and lane + 64 and ranks each against all of them with
// ballots over the bucket bits (most significant first: a lane below on a
// higher bit is less, and the equal set narrows), which gives the stable
// position; it writes order and inverse, scatters the buckets into LDS in
// sorted order, finds the first position of each bucket's run there (the
// leaders), and writes each run's tiles at the exclusive scan of the tile
// counts over the sorted positions. After the barrier every thread writes the
// counts and offsets of its experts (two binary searches of the sorted
// buckets) and zero-fills the descriptors past the last tile. The barrier
// orders LDS only. sb: R ints of
// LDS scratch; ntot: two ints of LDS, [0] the tiles written, [1] the valid
// ones (n_tiles), both readable by every thread on return.
template <typename Route>
__device__ __forceinline__ void plan_small_to(Route route, int R, int E, int tile, const PlanSmallOut& o, int* sb,
                                              int* ntot) {
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  if (wv == 0) {
    const bool v0 = lane < R, v1 = lane + 64 < R;
    int k0 = 0, k1 = 0;  // buckets: E collects invalid expert ids
    if (v0) {
      const int e = route(lane);
      k0 = (e < 0 || e >= E) ? E : e;
    }
    if (v1) {
      const int e = route(lane + 64);
      k1 = (e < 0 || e >= E) ? E : e;
    }
    const int nbits = 32 - __builtin_clz((unsigned)E);  // bucket ids 0..E
    const uint64_t in0 = __ballot(v0), in1 = __ballot(v1);
    uint64_t eq00 = in0, eq01 = in1, eq10 = in0, eq11 = in1;  // eqAB: routes of half B equal so far to my A key
    uint64_t lt00 = 0, lt01 = 0, lt10 = 0, lt11 = 0;          // ... and below it
    const bool two = R > 64;  // the second half holds routes (else its masks stay 0: skipped)
    for (int b = nbits - 1; b >= 0; --b) {
      const uint64_t m0 = __ballot((k0 >> b) & 1);
      const uint64_t s0 = ((k0 >> b) & 1) ? ~0ull : 0ull;
      lt00 |= eq00 & ~m0 & s0;
      eq00 &= ~(m0 ^ s0);
      if (two) {
        const uint64_t m1 = __ballot((k1 >> b) & 1);
        const uint64_t s1 = ((k1 >> b) & 1) ? ~0ull : 0ull;
        lt01 |= eq01 & ~m1 & s0;
        lt10 |= eq10 & ~m0 & s1;
        lt11 |= eq11 & ~m1 & s1;
        eq01 &= ~(m1 ^ s0);
        eq10 &= ~(m0 ^ s1);
        eq11 &= ~(m1 ^ s1);
      }
    }
    const uint64_t below = (1ull << lane) - 1ull;
    const int p0 = __popcll(lt00) + __popcll(lt01) + __popcll(eq00 & below);
    const int p1 = __popcll(lt10) + __popcll(lt11) + __popcll(eq10) + __popcll(eq11 & below);
    if (v0) {
      if (o.order) o.order[p0] = lane;
      if (o.l_order) o.l_order[p0] = lane;
      if (o.inverse) o.inverse[lane] = p0;
      sb[p0] = k0;
    }
    if (v1) {
      if (o.order) o.order[p1] = lane + 64;
      if (o.l_order) o.l_order[p1] = lane + 64;
      if (o.inverse) o.inverse[lane + 64] = p1;
      sb[p1] = k1;
    }
    // the sorted view: lane q holds positions q and q + 64
    const int b0 = v0 ? sb[lane] : -1, b1 = v1 ? sb[lane + 64] : -1;
    const int pb0 = sb[lane > 0 ? lane - 1 : 0], pb1 = sb[lane + 63];
    const bool l0 = v0 && (lane == 0 || pb0 != b0), l1 = v1 && pb1 != b1;  // first position of a run
    const uint64_t L0 = __ballot(l0), L1 = __ballot(l1);
    auto run_end = [&](int q) {  // the next leader after position q, or R
      if (q < 64) {
        const uint64_t m = q < 63 ? L0 >> (q + 1) : 0ull;
        if (m) return q + 1 + __builtin_ctzll(m);
        return L1 ? 64 + __builtin_ctzll(L1) : R;
      }
      const int t = q - 64;
      const uint64_t m = t < 63 ? L1 >> (t + 1) : 0ull;
      return m ? q + 1 + __builtin_ctzll(m) : R;
    };
    const int c0 = l0 ? run_end(lane) - lane : 0, c1 = l1 ? run_end(lane + 64) - (lane + 64) : 0;
    const int n0 = (c0 + tile - 1) / tile, n1 = (c1 + tile - 1) / tile;
    int x0 = n0, x1 = n1;  // inclusive scans over the lanes
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const int y0 = __shfl_up(x0, d, 64), y1 = __shfl_up(x1, d, 64);
      if (lane >= d) {
        x0 += y0;
        x1 += y1;
      }
    }
    const int tot0 = __shfl(x0, 63, 64), total = tot0 + __shfl(x1, 63, 64);
    const int tb0 = x0 - n0, tb1 = tot0 + x1 - n1;
    auto put = [&](int ti, int e, int off, int cnt) {
      if (o.te) {
        o.te[ti] = e;
        o.to[ti] = off;
        o.tc[ti] = cnt;
      }
      if (o.l_te) {
        o.l_te[ti] = e;
        o.l_to[ti] = off;
        o.l_tc[ti] = cnt;
      }
    };
    for (int i = 0; i < n0; ++i) put(tb0 + i, b0 < E ? b0 : -1, lane + i * tile, min(tile, c0 - i * tile));
    for (int i = 0; i < n1; ++i) put(tb1 + i, b1 < E ? b1 : -1, lane + 64 + i * tile, min(tile, c1 - i * tile));
    // the invalid routes' run sorts last: its tiles are not counted
    const uint64_t bad0 = __ballot(l0 && b0 == E), bad1 = __ballot(l1 && b1 == E);
    const int nbad = bad1 ? __shfl(n1, __builtin_ctzll(bad1), 64) : bad0 ? __shfl(n0, __builtin_ctzll(bad0), 64) : 0;
    if (lane == 0) {
      if (o.n_tiles) o.n_tiles[0] = total - nbad;
      ntot[0] = total;
      ntot[1] = total - nbad;
    }
  }
  // LDS only: the global writes are for later launches, so no wave waits here for their completion
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
  const int total = ntot[0];
  if (o.counts) {
    for (int e = tid; e < E; e += PLAN_THREADS) {
      int lo = 0, hi = R;  // the first sorted position with bucket >= e
      while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        if (sb[mid] < e) lo = mid + 1;
        else hi = mid;
      }
      int lo2 = lo, hi2 = R;  // ... and > e
      while (lo2 < hi2) {
        const int mid = (lo2 + hi2) >> 1;
        if (sb[mid] <= e) lo2 = mid + 1;
        else hi2 = mid;
      }
      o.offsets[e] = lo;
      o.counts[e] = lo2 - lo;
    }
  }
  if (o.te) {
    for (int ti = total + tid; ti < o.max_tiles; ti += PLAN_THREADS) {
      o.te[ti] = 0;
      o.to[ti] = 0;
      o.tc[ti] = 0;
    }
  }
}

// plan_small_to with every output in global memory and PlanLds as scratch.
template <typename Route>
__device__ __forceinline__ void plan_small(Route route, int R, int E, int tile, int32_t* order, int32_t* inverse,
                                           int32_t* counts, int32_t* offsets, int32_t* te, int32_t* to, int32_t* tc,
                                           int max_tiles, int32_t* n_tiles_out, PlanLds& L) {
  const PlanSmallOut o{order, inverse, counts, offsets, te, to, tc, n_tiles_out, max_tiles,
                       nullptr, nullptr, nullptr, nullptr};
  plan_small_to(route, R, E, tile, o, L.cnt, L.wtot[0]);
}

}  // namespace keep
