// Device helpers shared by the MoE decode kernels (moe.hip, moe_i8.hip).
#pragma once
#include "common.h"

namespace keep {

// SwiGLU with the optional clamp of LimitedSwiGLU
// (src/ramp/models/deepseek_v4_flash_adapter.py:962-986): for limit > 0 the
// gate is clamped above at limit and the up projection to [-limit, limit].
__device__ __forceinline__ float silu_mul(float g, float u, float limit) {
  if (limit > 0.f) {
    g = fminf(g, limit);
    u = fminf(fmaxf(u, -limit), limit);
  }
  return g / (1.f + __expf(-g)) * u;
}

// Force a value into a vector register (keeps the load it feeds a vector load).
__device__ __forceinline__ uint32_t vreg(uint32_t v) {
  asm volatile("" : "+v"(v));
  return v;
}

// Scales are fetched branch-free as the aligned 32-bit word holding element i
// (one vector load whatever the dtype; an aligned word never crosses a page)
// and converted after the LDS barrier.
typedef uint32_t ScaleRaw;
__device__ __forceinline__ ScaleRaw scale_raw(const void* p, int dt, uint32_t i) {
  const uint32_t off = vreg(dt == KEEP_F32 ? i * 4u : i * 2u);
  return *(const uint32_t*)((const char*)p + (off & ~3u));
}
__device__ __forceinline__ float scale_cvt(ScaleRaw word, int dt, uint32_t i) {
  const uint32_t h = (word >> ((i & 1u) * 16u)) & 0xffffu;
  const float f16 = (float)__builtin_bit_cast(_Float16, (uint16_t)h);
  const float b16 = __uint_as_float(h << 16);
  const float f32 = __uint_as_float(word);
  return dt == KEEP_F32 ? f32 : (dt == KEEP_BF16 ? b16 : f16);
}

}  // namespace keep
