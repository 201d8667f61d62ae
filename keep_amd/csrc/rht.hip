// Random-sign Walsh-Hadamard transform of activation rows on gfx950.
//
// forward:  y = FWHT(x * s) * (1 / sqrt(n))     (reference apply_rht_np, src/keep/quant/rht.py:51-57)
// inverse:  y = (FWHT(x) * (1 / sqrt(n))) * s   (reference apply_inverse_rht_np, rht.py:60-66)
//
// The butterflies are float32 and run in the reference's stage order (width 1,
// 2, 4, ..., n/2; pair (i, i + width) -> (a + b, a - b), rht.py:34-48), so the
// float32 result is bit-identical to the reference's numpy path whatever the
// schedule: every butterfly sees the same two fp32 inputs.
//
// One block per row, n / 16 threads, 16 values per thread in registers. The
// log2(n) stages are taken four index bits per pass: in pass p a thread holds
// the 16 values whose index bits [4p, 4p + 4) vary (the other bits fixed by
// the thread), runs those stages in registers, and the values move through a
// padded LDS row to the next pass's arrangement. The first pass loads 16
// consecutive values (two or four 16-byte loads), the last stores straight to
// HBM. HBM-bound: n * (in + out bytes) per row.
#include <cmath>

#include "common.h"

using namespace keep;

namespace {

constexpr int RHT_MAX_LOG = 13;  // n <= 8192: 16 values x 512 threads, 34 KiB of LDS

__device__ __forceinline__ uint32_t lds_pad(uint32_t i) { return i + (i >> 4); }

// index of value m (0..15) of thread t in the pass over bits [lo, lo + nb)
template <int L>
__device__ __forceinline__ uint32_t pass_index(uint32_t t, uint32_t m, int lo, int nb) {
  const uint32_t free = (t << (4 - nb)) | (m >> nb);
  const uint32_t v = m & ((1u << nb) - 1u);
  return (free & ((1u << lo) - 1u)) | (v << lo) | ((free >> lo) << (lo + nb));
}

__device__ __forceinline__ void load16(const void* x, int dt, size_t off, float r[16]) {
  if (dt == KEEP_F32) {
    const float4* p = (const float4*)((const float*)x + off);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const float4 v = p[q];
      r[4 * q] = v.x; r[4 * q + 1] = v.y; r[4 * q + 2] = v.z; r[4 * q + 3] = v.w;
    }
  } else {
    const uint4* p = (const uint4*)((const uint16_t*)x + off);
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const uint4 v = p[q];
      const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const uint16_t lo = (uint16_t)(w[u] & 0xFFFFu), hi = (uint16_t)(w[u] >> 16);
        if (dt == KEEP_BF16) {
          r[8 * q + 2 * u] = to_float(bf16s{lo});
          r[8 * q + 2 * u + 1] = to_float(bf16s{hi});
        } else {
          r[8 * q + 2 * u] = to_float(__builtin_bit_cast(_Float16, lo));
          r[8 * q + 2 * u + 1] = to_float(__builtin_bit_cast(_Float16, hi));
        }
      }
    }
  }
}

__device__ __forceinline__ void store1(void* out, int dt, size_t i, float v) {
  if (dt == KEEP_F32) ((float*)out)[i] = v;
  else if (dt == KEEP_BF16) ((uint16_t*)out)[i] = from_float<bf16s>(v).bits;
  else ((_Float16*)out)[i] = (_Float16)v;
}

template <int L, bool INV>
__global__ __launch_bounds__(512) void k_rht(const void* x, int xdt, const float* signs, void* out, int odt,
                                            float scale) {
  constexpr uint32_t N = 1u << L;
  constexpr int PASSES = (L + 3) / 4;
  __shared__ float s[N + N / 16];
  const uint32_t t = threadIdx.x;
  const size_t row = (size_t)blockIdx.x * N;
  float r[16];
  load16(x, xdt, row + (size_t)t * 16, r);
  if (!INV && signs) {
    const float4* sp = (const float4*)(signs + t * 16);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const float4 v = sp[q];
      r[4 * q] *= v.x; r[4 * q + 1] *= v.y; r[4 * q + 2] *= v.z; r[4 * q + 3] *= v.w;
    }
  }
#pragma unroll
  for (int p = 0; p < PASSES; ++p) {
    const int lo = 4 * p;
    const int nb = L - lo < 4 ? L - lo : 4;
    if (p > 0) {
#pragma unroll
      for (int m = 0; m < 16; ++m) r[m] = s[lds_pad(pass_index<L>(t, m, lo, nb))];
    }
#pragma unroll
    for (int b = 0; b < nb; ++b) {
#pragma unroll
      for (int m = 0; m < 16; ++m) {
        if (m & (1 << b)) continue;
        const float a = r[m], c = r[m | (1 << b)];
        r[m] = a + c;
        r[m | (1 << b)] = a - c;
      }
    }
    if (p + 1 < PASSES) {
      if (p > 0) __syncthreads();  // every read of the previous arrangement done
#pragma unroll
      for (int m = 0; m < 16; ++m) s[lds_pad(pass_index<L>(t, m, lo, nb))] = r[m];
      __syncthreads();
    } else {
#pragma unroll
      for (int m = 0; m < 16; ++m) {
        const uint32_t i = pass_index<L>(t, m, lo, nb);
        float v = r[m] * scale;
        if (INV && signs) v *= signs[i];
        store1(out, odt, row + i, v);
      }
    }
  }
}

template <int L>
void launch_rht(const void* x, int xdt, const float* signs, int inverse, int64_t T, void* out, int odt, float scale,
                hipStream_t s) {
  const dim3 grid((unsigned)T), blk((1u << L) / 16);
  if (inverse) hipLaunchKernelGGL((k_rht<L, true>), grid, blk, 0, s, x, xdt, signs, out, odt, scale);
  else hipLaunchKernelGGL((k_rht<L, false>), grid, blk, 0, s, x, xdt, signs, out, odt, scale);
}

}  // namespace

extern "C" int keep_rht(const void* x, int x_dtype, const float* signs, int inverse, int64_t T, int64_t n, void* out,
                        int out_dtype, void* stream) {
  KEEP_REQUIRE(dtype_ok(x_dtype) && dtype_ok(out_dtype), "bad dtype enum");
  KEEP_REQUIRE(n > 0 && (n & (n - 1)) == 0, "RHT dimension must be a positive power of two");
  KEEP_REQUIRE(T >= 0 && T <= 0x7FFFFFFF, "row count out of range");
  if (n < 16 || n > (1 << RHT_MAX_LOG)) {
    set_error("keep_rht serves 16 <= n <= 8192");
    return KEEP_EUNSUPPORTED;
  }
  if (T == 0) return KEEP_OK;
  KEEP_REQUIRE(x && out, "null pointer argument");
  KEEP_REQUIRE(aligned(x, 16) && (!signs || aligned(signs, 16)), "x and signs must be 16-byte aligned");
  KEEP_REQUIRE(x != out, "keep_rht does not run in place");
  const float scale = (float)(1.0 / std::sqrt((double)n));
  const hipStream_t s = (hipStream_t)stream;
  int L = 0;
  while ((int64_t(1) << L) < n) ++L;
  switch (L) {
    case 4: launch_rht<4>(x, x_dtype, signs, inverse, T, out, out_dtype, scale, s); break;
    case 5: launch_rht<5>(x, x_dtype, signs, inverse, T, out, out_dtype, scale, s); break;
    case 6: launch_rht<6>(x, x_dtype, signs, inverse, T, out, out_dtype, scale, s); break;
    case 7: launch_rht<7>(x, x_dtype, signs, inverse, T, out, out_dtype, scale, s); break;
    case 8: launch_rht<8>(x, x_dtype, signs, inverse, T, out, out_dtype, scale, s); break;
    case 9: launch_rht<9>(x, x_dtype, signs, inverse, T, out, out_dtype, scale, s); break;
    case 10: launch_rht<10>(x, x_dtype, signs, inverse, T, out, out_dtype, scale, s); break;
    case 11: launch_rht<11>(x, x_dtype, signs, inverse, T, out, out_dtype, scale, s); break;
    case 12: launch_rht<12>(x, x_dtype, signs, inverse, T, out, out_dtype, scale, s); break;
    default: launch_rht<13>(x, x_dtype, signs, inverse, T, out, out_dtype, scale, s); break;
  }
  return launch_status("keep_rht");
}
