// Device route plan kernel (the plan itself is plan_small / plan_block in plan_dev.h).
#include "plan_dev.h"

namespace keep {

__global__ __launch_bounds__(PLAN_THREADS) void k_route_plan(const int32_t* rhs, int R, int E, int tile,
                                                             int32_t* order, int32_t* inverse, int32_t* counts,
                                                             int32_t* offsets, int32_t* te, int32_t* to, int32_t* tc,
                                                             int max_tiles, int32_t* n_tiles_out) {
  __shared__ PlanLds L;
  auto route = [&](int r) { return rhs[r]; };
  if (R <= PLAN_SMALL_R)
    plan_small(route, R, E, tile, order, inverse, counts, offsets, te, to, tc, max_tiles, n_tiles_out, L);
  else
    plan_block(route, R, E, tile, order, inverse, counts, offsets, te, to, tc, max_tiles, n_tiles_out, L);
}

}  // namespace keep

using namespace keep;

extern "C" int keep_route_plan(const int32_t* rhs, int64_t R, int64_t E, int64_t tile, int32_t* order,
                               int32_t* inverse, int32_t* counts, int32_t* offsets, int32_t* tile_expert,
                               int32_t* tile_offset, int32_t* tile_count, int64_t max_tiles, int32_t* n_tiles_out,
                               void* stream) {
  KEEP_REQUIRE_DIMS(R, E, tile, max_tiles);
  KEEP_REQUIRE(R >= 0 && R <= 0x7fffffffLL, "bad route count");
  KEEP_REQUIRE(E >= 1 && E <= PLAN_MAX_E, "E must be in 1..%d", PLAN_MAX_E);
  KEEP_REQUIRE(tile >= 1 && tile <= 4096, "tile must be in 1..4096");
  KEEP_REQUIRE(max_tiles >= (R + tile - 1) / tile + E, "max_tiles must be >= ceil(R/tile) + E");
  KEEP_REQUIRE(max_tiles <= 0x7fffffffLL, "max_tiles too large");
  KEEP_REQUIRE((R == 0 || (rhs && order && inverse)) && counts && offsets && tile_expert && tile_offset &&
                   tile_count && n_tiles_out,
               "null pointer argument");
  hipLaunchKernelGGL(k_route_plan, dim3(1), dim3(PLAN_THREADS), 0, (hipStream_t)stream, rhs, (int)R, (int)E,
                     (int)tile, order, inverse, counts, offsets, tile_expert, tile_offset, tile_count, (int)max_tiles,
                     n_tiles_out);
  return launch_status("keep_route_plan");
}
