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
//
// keep_rmsnorm_quant_rht fuses the steps in front of the routed experts into
// the same row pass: RMSNorm, block-wise FP8 e4m3 activation quantisation
// (the act_quant of scripts/runpod/v41_reap/torch_kernel.py:40-53, whose
// values the serving step feeds to the experts, omlx_lattice.py:332,357) and
// the forward RHT.
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

// The passes over the 16 values r[] of thread t (forward signs applied first
// unless INV), then the store of row `row`.
template <int L, bool INV>
__device__ __forceinline__ void rht_core(float (&r)[16], float* s, uint32_t t, const float* signs, void* out, int odt,
                                         size_t row, float scale) {
  constexpr int PASSES = (L + 3) / 4;
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

template <int L, bool INV>
__global__ __launch_bounds__(512) void k_rht(const void* x, int xdt, const float* signs, void* out, int odt,
                                            float scale) {
  constexpr uint32_t N = 1u << L;
  __shared__ float s[N + N / 16];
  const uint32_t t = threadIdx.x;
  const size_t row = (size_t)blockIdx.x * N;
  float r[16];
  load16(x, xdt, row + (size_t)t * 16, r);
  rht_core<L, INV>(r, s, t, signs, out, odt, row, scale);
}

// ------------------------------------------------------------------ RMSNorm + FP8 act-quant (+ RHT)

// v rounded to the row dtype (fp32 rows: unchanged).
__device__ __forceinline__ float round_to(float v, int dt) {
  if (dt == KEEP_BF16) return to_float(from_float<bf16s>(v));
  if (dt == KEEP_F16) return (float)(_Float16)v;
  return v;
}

// Nearest FP8 e4m3fn value (ties to even) of v, |v| <= 448: 3 mantissa bits
// for |v| >= 2^-6, a fixed quantum of 2^-9 below (the subnormals).
__device__ __forceinline__ float e4m3_round(float v) {
  const float a = fabsf(v);
  float q;
  if (a >= 0.015625f) {
    uint32_t b = __float_as_uint(a);
    b += 0x7FFFFu + ((b >> 20) & 1u);
    q = __uint_as_float(b & 0xFFF00000u);
  } else {
    q = __builtin_rintf(a * 512.f) * 0.001953125f;
  }
  return copysignf(q, v);
}

// 2^ceil(log2(v)) of a positive normal fp32 v.
__device__ __forceinline__ float pow2_ceil(float v) {
  const uint32_t b = __float_as_uint(v);
  const int e = (int)((b >> 23) & 0xFFu) - 127 + ((b & 0x7FFFFFu) != 0u ? 1 : 0);
  return __uint_as_float((uint32_t)(e + 127) << 23);
}

// One row per block, N / 16 threads of 16 consecutive values:
//   y  = round_T(gamma * (x * (1 / sqrt(mean(x^2) + eps))))      (RMSNorm, fp32 math)
//   q  = round_T(e4m3(clamp(y / s, +-448)) * s) per qblock values, s = max(amax, 1e-4) / 448
//        (2^ceil(log2 s) with pow2), qblock = 0: q = y
//   out = RHT(q, signs) when signs are given, else q.
// `normed` (optional) receives y in the row dtype.
template <int L, bool RHT>
__global__ __launch_bounds__(512) void k_norm_quant(const void* x, int xdt, const void* gamma, int gdt, float eps,
                                                   int qblock, int pow2, const float* signs, void* normed, void* out,
                                                   int odt, float scale) {
  constexpr uint32_t N = 1u << L;
  constexpr uint32_t NT = N / 16;
  constexpr uint32_t NW = (NT + 63) / 64;
  __shared__ float s[N + N / 16];
  __shared__ float part[NW];
  const uint32_t t = threadIdx.x;
  const size_t row = (size_t)blockIdx.x * N;
  float r[16], g[16];
  load16(x, xdt, row + (size_t)t * 16, r);
  if (gamma) load16(gamma, gdt, (size_t)t * 16, g);
  float ss = 0.f;
#pragma unroll
  for (int m = 0; m < 16; ++m) ss = fmaf(r[m], r[m], ss);
  for (int o = (NT < 64 ? NT : 64) / 2; o > 0; o >>= 1) ss += __shfl_xor(ss, o, 64);  // live lanes only
  if (NT >= 64) {
    if ((t & 63u) == 0u) part[t >> 6] = ss;
    __syncthreads();
    ss = 0.f;
#pragma unroll
    for (uint32_t w = 0; w < NW; ++w) ss += part[w];
  }
  const float inv = 1.f / sqrtf(ss / (float)N + eps);
#pragma unroll
  for (int m = 0; m < 16; ++m) {
    const float v = r[m] * inv;
    r[m] = round_to(gamma ? g[m] * v : v, xdt);
  }
  if (normed) {
#pragma unroll
    for (int m = 0; m < 16; ++m) store1(normed, xdt, row + (size_t)t * 16 + m, r[m]);
  }
  if (qblock > 0) {
    float amax = 0.f;
#pragma unroll
    for (int m = 0; m < 16; ++m) amax = fmaxf(amax, fabsf(r[m]));
    for (int o = 1; o < qblock / 16; o <<= 1) amax = fmaxf(amax, __shfl_xor(amax, o, 64));
    float sc = fmaxf(amax, 1e-4f) * (1.f / 448.f);
    if (pow2) sc = pow2_ceil(sc);
#pragma unroll
    for (int m = 0; m < 16; ++m) {
      const float q = e4m3_round(fminf(fmaxf(r[m] / sc, -448.f), 448.f));
      r[m] = round_to(q * sc, xdt);
    }
  }
  if constexpr (RHT) {
    rht_core<L, false>(r, s, t, signs, out, odt, row, scale);
  } else {
#pragma unroll
    for (int m = 0; m < 16; ++m) store1(out, odt, row + (size_t)t * 16 + m, r[m]);
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
  KEEP_REQUIRE_DIMS(T, n);
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

namespace {

template <int L>
void launch_norm_quant(const void* x, int xdt, const void* gamma, int gdt, float eps, int qblock, int pow2,
                       const float* signs, void* normed, int64_t T, void* out, int odt, float scale, hipStream_t s) {
  const dim3 grid((unsigned)T), blk((1u << L) / 16);
  if (signs)
    hipLaunchKernelGGL((k_norm_quant<L, true>), grid, blk, 0, s, x, xdt, gamma, gdt, eps, qblock, pow2, signs, normed,
                       out, odt, scale);
  else
    hipLaunchKernelGGL((k_norm_quant<L, false>), grid, blk, 0, s, x, xdt, gamma, gdt, eps, qblock, pow2, signs,
                       normed, out, odt, scale);
}

}  // namespace

extern "C" int keep_rmsnorm_quant_rht(const void* x, int x_dtype, int64_t T, int64_t n, const void* gamma,
                                      int gamma_dtype, float eps, int64_t quant_block, int pow2_scales,
                                      const float* signs, void* normed, void* out, int out_dtype, void* stream) {
  KEEP_REQUIRE_DIMS(T, n, quant_block);
  KEEP_REQUIRE(dtype_ok(x_dtype) && dtype_ok(out_dtype) && (!gamma || dtype_ok(gamma_dtype)), "bad dtype enum");
  KEEP_REQUIRE(n >= 64 && n <= (1 << RHT_MAX_LOG) && (n & (n - 1)) == 0,
               "keep_rmsnorm_quant_rht serves power-of-two rows of 64..8192 values, got %lld", (long long)n);
  KEEP_REQUIRE(quant_block == 0 || (quant_block >= 16 && quant_block <= 1024 && quant_block <= n &&
                                    (quant_block & (quant_block - 1)) == 0),
               "quant_block must be 0 or a power of two in 16..min(1024, n), got %lld", (long long)quant_block);
  KEEP_REQUIRE(eps >= 0.f, "eps must be non-negative");
  KEEP_REQUIRE(T >= 0 && T <= 0x7FFFFFFF, "row count out of range");
  if (T == 0) return KEEP_OK;
  KEEP_REQUIRE(x && out, "null pointer argument");
  KEEP_REQUIRE(aligned(x, 16) && aligned(out, 16) && (!gamma || aligned(gamma, 16)) &&
                   (!signs || aligned(signs, 16)) && (!normed || aligned(normed, 16)),
               "x, gamma, signs, normed and out must be 16-byte aligned");
  KEEP_REQUIRE(x != out && x != normed, "keep_rmsnorm_quant_rht does not run in place");
  const float scale = (float)(1.0 / std::sqrt((double)n));
  const hipStream_t s = (hipStream_t)stream;
  const int q = (int)quant_block;
  int L = 0;
  while ((int64_t(1) << L) < n) ++L;
#define NQ(LL) launch_norm_quant<LL>(x, x_dtype, gamma, gamma_dtype, eps, q, pow2_scales, signs, normed, T, out, \
                                     out_dtype, scale, s)
  switch (L) {
    case 6: NQ(6); break;
    case 7: NQ(7); break;
    case 8: NQ(8); break;
    case 9: NQ(9); break;
    case 10: NQ(10); break;
    case 11: NQ(11); break;
    case 12: NQ(12); break;
    default: NQ(13); break;
  }
#undef NQ
  return launch_status("keep_rmsnorm_quant_rht");
}
