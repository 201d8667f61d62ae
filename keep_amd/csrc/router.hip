// Residency-biased dual top-k router: one wave64 per token.
//
// Each lane holds experts e = lane + 64*i. One evaluation of the score
// function feeds two selections: served (scores + bias_served, absent experts
// carry bias <= -1e30 and get weight 0) and demand (scores + bias_demand, the
// unmasked pool). Selection is k rounds of a wave arg-max with the total
// order "larger key, then lower index"; NaN keys rank as -inf. With a slot
// map (a pool of S slots smaller than the expert count) the served outputs
// are the experts' slots, as the serving router's (omlx_lattice.py:77-97,
// slot[b k + j] = slot_of[chosen[j]]); the demand outputs stay expert ids.
#include "route_dev.h"

namespace keep {

template <int PER>
__global__ __launch_bounds__(256) void k_router(const float* logits, int T, int E, int k, const float* bias_s,
                                                const float* bias_d, int func, int renorm, float route_scale,
                                                float tau, const int32_t* slot_map, int S, int32_t* idx, float* w,
                                                int32_t* want, float* want_score, uint8_t* admit) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  float z[PER], bs[PER], bd[PER];
  rt_load<PER>(logits + (int64_t)t * E, bias_s, bias_d, E, lane, z, bs, bd);
  const RouteLane r = rt_route<PER>(z, bs, bd, E, k, func, renorm, route_scale, tau, bias_d == bias_s, lane);
  int slot = r.expert;
  if (slot_map) {
    int sm[PER];
    rt_load_slots<PER>(slot_map, E, lane, sm);
    slot = rt_slot_of<PER>(sm, r.valid ? r.expert : -1, E, S);
  }
  if (!r.valid) return;
  const int64_t o = (int64_t)t * k + (lane < 32 ? lane : lane - 32);
  if (lane < 32) {
    idx[o] = slot;
    w[o] = r.value;
  } else {
    if (want) want[o] = r.expert;
    if (want_score) want_score[o] = r.value;
    if (admit) admit[o] = r.admit;
  }
}

}  // namespace keep

using namespace keep;

extern "C" int keep_router_dual_topk(const float* logits, int64_t T, int64_t E, int64_t k, const float* bias_served,
                                     const float* bias_demand, int score_func, int renormalize, float route_scale,
                                     float tau, const int32_t* slot_map, int64_t num_slots, int32_t* idx, float* w,
                                     int32_t* want, float* want_score, uint8_t* admit, void* stream) {
  KEEP_REQUIRE_DIMS(T, E, k, num_slots);
  KEEP_REQUIRE(T >= 0, "T must be >= 0");
  KEEP_REQUIRE(E >= 1 && E <= 64 * RT_MAX_PER_LANE, "E must be in 1..%d, got %lld", 64 * RT_MAX_PER_LANE,
               (long long)E);
  KEEP_REQUIRE(k >= 1 && k <= 32 && k <= E, "k must be in 1..min(32, E), got %lld", (long long)k);
  KEEP_REQUIRE(score_func >= 0 && score_func <= 2, "bad score_func %d", score_func);
  if (T == 0) return KEEP_OK;
  KEEP_REQUIRE(T <= 0x7fffffffLL, "T too large");
  KEEP_REQUIRE(logits && idx && w, "logits, idx and w must be non-null");
  KEEP_REQUIRE(!slot_map || (num_slots >= 1 && num_slots <= 0x7fffffffLL), "num_slots must be positive");
  const unsigned blocks = (unsigned)((T + 3) / 4);
  hipStream_t s = (hipStream_t)stream;
  const int per = (int)((E + 63) / 64);
#define KEEP_ROUTER_LAUNCH(P)                                                                                   \
  hipLaunchKernelGGL((k_router<P>), dim3(blocks), dim3(256), 0, s, logits, (int)T, (int)E, (int)k, bias_served, \
                     bias_demand, score_func, renormalize, route_scale, tau, slot_map, (int)num_slots, idx, w, want, \
                     want_score, admit)
  if (per <= 1) KEEP_ROUTER_LAUNCH(1);
  else if (per <= 2) KEEP_ROUTER_LAUNCH(2);
  else if (per <= 4) KEEP_ROUTER_LAUNCH(4);
  else if (per <= 6) KEEP_ROUTER_LAUNCH(6);
  else if (per <= 8) KEEP_ROUTER_LAUNCH(8);
  else KEEP_ROUTER_LAUNCH(16);
#undef KEEP_ROUTER_LAUNCH
  return launch_status("keep_router_dual_topk");
}
