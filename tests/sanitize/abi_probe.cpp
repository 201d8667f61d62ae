// Argument probes of every C-ABI entry point, built with the library's host
// code under AddressSanitizer and UndefinedBehaviorSanitizer (no GPU needed):
// each entry point is called with all-zero / all-null arguments, with -1 /
// NaN sizes, and with huge sizes; it must return KEEP_OK or KEEP_EINVAL
// without touching memory it was not given and without undefined behaviour
// (signed overflow in a size check, a shift past the width, ...). Host-only
// entry points are then called with valid buffers and checked.
#include <cmath>
#include <cstdio>
#include <cstring>
#include <limits>
#include <type_traits>

#include "keep_amd.h"

template <class T>
T fill(int mode) {
  if constexpr (std::is_pointer_v<T>) {
    return nullptr;
  } else if constexpr (std::is_floating_point_v<T>) {
    return mode == 0 ? T(0) : mode == 1 ? T(NAN) : T(1e30);
  } else {
    if (mode == 0) return T(0);
    if (mode == 1) return T(-1);
    return std::numeric_limits<T>::max() / 3;
  }
}

static int failures = 0;

template <class R, class... A>
void probe(const char* name, R (*f)(A...)) {
  for (int mode = 0; mode < 3; ++mode) {
    R r = f(fill<A>(mode)...);
    if constexpr (std::is_same_v<R, int>) {
      if (r != KEEP_OK && r != KEEP_EINVAL) {
        std::printf("FAIL %s mode %d returned %d: %s\n", name, mode, r, keep_last_error());
        ++failures;
      }
    }
  }
}

#define PROBE(f) probe(#f, &f)

int main() {
  PROBE(keep_e8p_decode);
  PROBE(keep_e8_1bit_decode);
  PROBE(keep_vq_encode);
  PROBE(keep_group_absmax);
  PROBE(keep_vq_matvec);
  PROBE(keep_e8_1bit_matvec);
  PROBE(keep_vq_matvec_tiles);
  PROBE(keep_router_dual_topk);
  PROBE(keep_route_plan);
  PROBE(keep_e8p_prepare);
  PROBE(keep_moe_decode);
  PROBE(keep_moe_gateup);
  PROBE(keep_moe_down);
  PROBE(keep_moe_layer_supported);
  PROBE(keep_moe_layer);
  PROBE(keep_moe_layer_noalloc);
  PROBE(keep_moe_layer1_workspace_bytes);
  PROBE(keep_moe_layer1_status);
  PROBE(keep_moe_layer1);
  PROBE(keep_moe_layer1_nested);
  PROBE(keep_e8_1bit_image);
  PROBE(keep_moe_layer_nested);
  PROBE(keep_moe_tiles_workspace_bytes);
  PROBE(keep_moe_tiles_supported);
  PROBE(keep_moe_tiles);
  PROBE(keep_moe_tiles_layer);
  PROBE(keep_vq_grouped_gemm_q8_workspace_bytes);
  PROBE(keep_vq_grouped_gemm_q8);
  PROBE(keep_vq_grouped_swiglu_q8);
  PROBE(keep_vq_grouped_swiglu_nested_q8);
  PROBE(keep_vq_grouped_gemm_nested_q8);
  PROBE(keep_route_combine);
  PROBE(keep_rht);
  PROBE(keep_rmsnorm_quant_rht);
  PROBE(keep_moe_combine_add);
  // the spin budget: out of range rejected, in range set and read back
  uint32_t prev = 0;
  if (keep_moe_layer1_set_spin_ticks(200000000u, &prev) != KEEP_EINVAL) ++failures;
  if (keep_moe_layer1_set_spin_ticks(7u, &prev) != KEEP_OK || prev != 20000u) ++failures;
  if (keep_moe_layer1_set_spin_ticks(20000u, &prev) != KEEP_OK || prev != 7u) ++failures;
  // host-only entry points on valid buffers
  uint32_t table[256];
  std::memset(table, 0, sizeof table);
  if (keep_e8p_packed_abs_grid(table) != KEEP_OK || table[0] == 0) ++failures;
  if (keep_e8_1bit_packed(table) != KEEP_OK || table[0] == 0) ++failures;
  if (keep_abi_version() < 1 || keep_e8p_prepared_bytes() <= 0 || keep_e8_1bit_image_bytes() <= 0) ++failures;
  if (keep_moe_layer1_workspace_bytes(6, 2048) != 256 + 4 * 6 * 2048) ++failures;
  if (keep_moe_layer_supported(384, 4096, 2048, 6, 4096, 2048) != 1) ++failures;
  if (std::strlen(keep_last_error()) == 0) ++failures;  // the probes above left a message
  std::printf("%s: %d failures\n", failures ? "FAIL" : "ok", failures);
  return failures ? 1 : 0;
}
