// Host entry points of the routed decode layer (keep_moe_layer, its
// allocation-free form) and of the decode tables (keep_e8p_prepare). The
// kernels are in moe_i8.hip (two launches) and layer.hip (one launch).
#include <mutex>

#include "common.h"
#include "moe_dev.h"
#include "q8_dev.h"
#include "route_dev.h"

namespace keep {

// int8 matrix-core layer (moe_i8.hip)
void tq_build(const uint32_t* table, void* prepared, hipStream_t s);
bool moe_q_layer_supported(int64_t E, int64_t H, int64_t I, int64_t k, int64_t group_h, int64_t group_i);
int moe_q_layer_launch(const float* logits, const float* bias_s, const float* bias_d, int func, int renorm,
                        float route_scale, float tau, const int32_t* slot_map, int64_t S, int64_t E, int64_t k,
                        const void* x, int x_dtype, int64_t H,
                        int64_t I, const uint16_t* gc, const void* gs, const uint16_t* uc, const void* us,
                        const uint16_t* dc, const void* ds, int sdt, int64_t group_h, int64_t group_i,
                        const void* prepared, float limit, int32_t* idx, float* w, int32_t* want, float* want_score,
                        uint8_t* admit, void* h, void* out, int odt, hipStream_t s, const struct MQNest* nest = nullptr);
constexpr int PREPARED_TOTAL = (int)TQR_OFFSET + TQR_BYTES;  // T and M, the flag word, the 64 KiB LDS image

}  // namespace keep

using namespace keep;

extern "C" int keep_e8p_prepare(const uint32_t* table, void* prepared, void* stream) {
  KEEP_REQUIRE(table && prepared, "table and prepared must be non-null");
  KEEP_REQUIRE(aligned(prepared, 16), "prepared must be 16-byte aligned");
  hipStream_t s = (hipStream_t)stream;
  tq_build(table, prepared, s);
  return launch_status("keep_e8p_prepare");
}

extern "C" int keep_e8p_prepared_bytes(void) { return PREPARED_TOTAL; }

extern "C" int keep_moe_layer_supported(int64_t E, int64_t H, int64_t I, int64_t k, int64_t group_size_h,
                                        int64_t group_size_i) {
  if (!::keep::dims_ok({E, H, I, k, group_size_h, group_size_i})) return 0;
  return moe_q_layer_supported(E, H, I, k, group_size_h, group_size_i) ? 1 : 0;
}

extern "C" int keep_moe_layer(const float* logits, const float* bias_served, const float* bias_demand, int score_func,
                              int renormalize, float route_scale, float tau, const int32_t* slot_map,
                              int64_t num_slots, int64_t E, int64_t k, const void* x,
                              int x_dtype, int64_t H, int64_t I, const uint16_t* gate_codes, const void* gate_scales,
                              const uint16_t* up_codes, const void* up_scales, const uint16_t* down_codes,
                              const void* down_scales, int scale_dtype, int64_t group_size_h, int64_t group_size_i,
                              const void* prepared, float swiglu_limit, int32_t* idx, float* w, int32_t* want,
                              float* want_score, uint8_t* admit, void* h_work, void* out, int out_dtype,
                              void* stream) {
  KEEP_REQUIRE_DIMS(num_slots, E, k, H, I, group_size_h, group_size_i);
  KEEP_REQUIRE(x_dtype == KEEP_F16 || x_dtype == KEEP_BF16, "activations must be fp16 or bf16");
  KEEP_REQUIRE(dtype_ok(scale_dtype) && dtype_ok(out_dtype), "bad dtype enum");
  KEEP_REQUIRE(score_func >= 0 && score_func <= 2, "bad score_func %d", score_func);
  KEEP_REQUIRE(group_size_h > 0 && H % group_size_h == 0 && group_size_i > 0 && I % group_size_i == 0,
               "bad group sizes");
  KEEP_REQUIRE(moe_q_layer_supported(E, H, I, k, group_size_h, group_size_i),
               "shape not served by the routed decode layer kernels (needs H = 4096, I a multiple of 512 up to "
               "2048, k <= 8, E <= 1024, scale groups of 256-element multiples)");
  KEEP_REQUIRE(!slot_map || (num_slots >= 1 && num_slots <= 1024), "num_slots must be in 1..1024");
  KEEP_REQUIRE(logits && x && gate_codes && gate_scales && up_codes && up_scales && down_codes && down_scales &&
                   prepared && idx && w && h_work && out,
               "null pointer argument");
  KEEP_REQUIRE(aligned(x, 16) && aligned(h_work, 16) && aligned(prepared, 16),
               "x, h_work and prepared must be 16-byte aligned");
  KEEP_REQUIRE(aligned(gate_codes, 16) && aligned(up_codes, 16) && aligned(down_codes, 8), "codes misaligned");
  moe_q_layer_launch(logits, bias_served, bias_demand, score_func, renormalize, route_scale, tau, slot_map, num_slots,
                      E, k, x, x_dtype, H, I, gate_codes, gate_scales, up_codes, up_scales, down_codes, down_scales, scale_dtype,
                      group_size_h, group_size_i, prepared, swiglu_limit, idx, w, want, want_score, admit, h_work,
                      out, out_dtype, (hipStream_t)stream);
  return launch_status("keep_moe_layer");
}

// ------------------------------------------------------------------ keep_moe_layer_noalloc
//
// keep_moe_layer with h in a file-scope device array instead of a caller's
// h_work, for callers that cannot allocate. Each GPU holds its own copy of
// the array for the life of the process; its address on a device is taken
// with hipGetSymbolAddress once, with that device current, and kept (the
// array's name in host code is not a device address). The gate/up launch
// writes every one of the k * I values before the down launch reads them,
// so nothing in it has to start at zero; calls that overlap on one GPU
// (two streams) share it and race.
constexpr int64_t NOALLOC_H_ELEMS = 12288;  // k * I bf16 values: 24 KiB, every shape keep_moe_layer serves
constexpr int NOALLOC_MAX_DEVICES = 64;
static __device__ __align__(256) uint16_t scratch[NOALLOC_H_ELEMS];

static std::mutex g_scratch_mu;
static void* g_scratch_ptr[NOALLOC_MAX_DEVICES];

// The current device's copy of `scratch`, or null (with the error recorded).
static void* noalloc_scratch() {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= NOALLOC_MAX_DEVICES) {
    set_error("keep_moe_layer_noalloc: no current device below %d", NOALLOC_MAX_DEVICES);
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
      set_error("keep_moe_layer_noalloc: hipGetSymbolAddress failed on device %d: %s", dev, hipGetErrorString(e));
      return nullptr;
    }
    g_scratch_ptr[dev] = p;
  }
  return g_scratch_ptr[dev];
}

extern "C" int keep_moe_layer_noalloc(const float* logits, const float* bias_served, const float* bias_demand,
                                      int score_func, int renormalize, float route_scale, float tau,
                                      const int32_t* slot_map, int64_t num_slots, int64_t E, int64_t k, const void* x, int x_dtype, int64_t H, int64_t I,
                                      const uint16_t* gate_codes, const void* gate_scales, const uint16_t* up_codes,
                                      const void* up_scales, const uint16_t* down_codes, const void* down_scales,
                                      int scale_dtype, int64_t group_size_h, int64_t group_size_i,
                                      const void* prepared, float swiglu_limit, int32_t* idx, float* w,
                                      int32_t* want, float* want_score, uint8_t* admit, void* out, int out_dtype,
                                      void* stream) {
  KEEP_REQUIRE_DIMS(num_slots, E, k, H, I, group_size_h, group_size_i);
  KEEP_REQUIRE(k >= 1 && I >= 1 && k * I <= NOALLOC_H_ELEMS,
               "keep_moe_layer_noalloc holds at most %lld SwiGLU values (k * I) in its static scratch, got %lld",
               (long long)NOALLOC_H_ELEMS, (long long)(k * I));
  void* h = noalloc_scratch();
  if (!h) return KEEP_ELAUNCH;
  return keep_moe_layer(logits, bias_served, bias_demand, score_func, renormalize, route_scale, tau, slot_map,
                        num_slots, E, k, x, x_dtype,
                        H, I, gate_codes, gate_scales, up_codes, up_scales, down_codes, down_scales, scale_dtype,
                        group_size_h, group_size_i, prepared, swiglu_limit, idx, w, want, want_score, admit, h, out,
                        out_dtype, stream);
}
