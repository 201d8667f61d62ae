// The step after the routed combine on gfx950: the shared expert's output and
// the residual stream added to the routed sum, rounded once to the output
// dtype,
//   out = round_out(residual + (routed + shared))     (fp32 sums, in that order)
// (src/ramp/models/deepseek_v4_flash_adapter.py:1784, where the MoE returns
// the routed sum plus the shared expert; the serving step adds the fp32
// routed sum inside the shared down projection and rounds to bf16,
// scripts/v41_build/omlx_lattice.py:374-388). Elementwise and HBM-bound:
// eight values per thread, 16-byte loads of the fp32 sums.
#include "common.h"

namespace keep {

__device__ __forceinline__ float ld_any(const void* p, int dt, size_t i) {
  if (dt == KEEP_F32) return ((const float*)p)[i];
  if (dt == KEEP_BF16) return to_float(bf16s{((const uint16_t*)p)[i]});
  return (float)((const _Float16*)p)[i];
}

__device__ __forceinline__ void st_any(void* p, int dt, size_t i, float v) {
  if (dt == KEEP_F32) ((float*)p)[i] = v;
  else if (dt == KEEP_BF16) ((uint16_t*)p)[i] = from_float<bf16s>(v).bits;
  else ((_Float16*)p)[i] = (_Float16)v;
}

__global__ __launch_bounds__(256) void k_combine_add(const float* routed, const void* shared, int sdt,
                                                     const void* residual, int rdt, size_t n, void* out, int odt) {
  const size_t i0 = ((size_t)blockIdx.x * blockDim.x + threadIdx.x) * 8;
  if (i0 >= n) return;
  float v[8];
  if (i0 + 8 <= n) {
    const float4 a = *(const float4*)(routed + i0), b = *(const float4*)(routed + i0 + 4);
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
  } else {
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = i0 + u < n ? routed[i0 + u] : 0.f;
  }
#pragma unroll
  for (int u = 0; u < 8; ++u) {
    if (i0 + u < n) {
      float acc = v[u];
      if (shared) acc += ld_any(shared, sdt, i0 + u);
      if (residual) acc = ld_any(residual, rdt, i0 + u) + acc;
      st_any(out, odt, i0 + u, acc);
    }
  }
}

}  // namespace keep

using namespace keep;

extern "C" int keep_moe_combine_add(const float* routed, const void* shared, int shared_dtype, const void* residual,
                                    int residual_dtype, int64_t n, void* out, int out_dtype, void* stream) {
  KEEP_REQUIRE_DIMS(n);
  KEEP_REQUIRE(dtype_ok(out_dtype) && (!shared || dtype_ok(shared_dtype)) && (!residual || dtype_ok(residual_dtype)),
               "bad dtype enum");
  KEEP_REQUIRE(n >= 0, "n must be >= 0");
  if (n == 0) return KEEP_OK;
  KEEP_REQUIRE(routed && out, "null pointer argument");
  KEEP_REQUIRE(aligned(routed, 16), "routed must be 16-byte aligned");
  const int64_t threads = (n + 7) / 8;
  const int64_t blocks = (threads + 255) / 256;
  KEEP_REQUIRE(blocks <= 0x7fffffffLL, "too many values");
  hipLaunchKernelGGL(k_combine_add, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream, routed, shared,
                     shared_dtype, residual, residual_dtype, (size_t)n, out, out_dtype);
  return launch_status("keep_moe_combine_add");
}
