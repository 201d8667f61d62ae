// Nearest-codeword encoders on gfx950: E8P (16-bit codes) and the 8-bit E8
// table, under an optional diagonal metric w (one shared [8], or one [8] per
// vector), the data-free RTN quantiser of src/keep/quant/rtn.py:270-318 and
// the weighted search of src/keep/vq/e8.py:367-539.
//
// The answer is defined as the exhaustive scan's: the codeword minimising
//   D = ((q0 + q1) + (q2 + q3)) + ((q4 + q5) + (q6 + q7)),  q_d = w_d ((v_d - c_d)^2)
// in double precision, ties to the lowest code. The E8P search is factored
// instead of scanning 65,536 codewords: for each shift (+1/4 with even stored
// sign parity, -1/4 with odd) and each of the 256 abs rows, the signs that
// follow the target's are optimal; an odd sign count is fixed by the single
// flip of least distance (ties: the lowest stored signs), and dimensions whose
// sign is free (w_d |t_d| = 0) take the lowest stored signs that satisfy the
// parity. Every candidate's D is the same tree over the same exact terms as
// the scan's (|v_d - c_d| = | |t_d| -+ a_d | exactly in double), so the two
// agree bit for bit except where distinct codewords' D differ by less than
// its rounding. One thread per vector; the 256 rows sit in LDS and every
// lane of a wave reads the same row (a broadcast). fp64 VALU-bound.
#include "common.h"

namespace keep {

constexpr int ENC_THREADS = 256;
__constant__ int kEncShuffle[8] = {0, 4, 1, 5, 2, 6, 3, 7};  // dim d reads packed nibble kEncShuffle[d]

__device__ __forceinline__ double enc_tree8(const double (&q)[8]) {
#pragma clang fp contract(off)
  return ((q[0] + q[1]) + (q[2] + q[3])) + ((q[4] + q[5]) + (q[6] + q[7]));
}

// The vector (divided by its scale, correctly rounded to fp32) and its weights.
template <int WMODE>
__device__ __forceinline__ void enc_load(const float* x, const float* w, const float* scales, int64_t vps, int64_t i,
                                         float (&v)[8], double (&wd)[8]) {
  const float4* xp = (const float4*)(x + i * 8);
  const float4 a = xp[0], b = xp[1];
  const float xs[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
  const double s = scales ? (double)scales[i / vps] : 1.0;
#pragma unroll
  for (int d = 0; d < 8; ++d) v[d] = scales ? (float)((double)xs[d] / s) : xs[d];
#pragma unroll
  for (int d = 0; d < 8; ++d) wd[d] = WMODE == 0 ? 1.0 : (double)w[(WMODE == 2 ? i * 8 : 0) + d];
}

template <int WMODE>
__global__ __launch_bounds__(ENC_THREADS) void k_e8p_encode(const float* x, int64_t n, const float* w,
                                                           const uint32_t* table, const float* scales, int64_t vps,
                                                           uint16_t* out) {
#pragma clang fp contract(off)
  __shared__ float sa[256][8];
  __shared__ uint32_t sneg[256];
  {
    const uint32_t word = table[threadIdx.x];
    uint32_t neg = 0;
#pragma unroll
    for (int d = 0; d < 8; ++d) {
      const int s = kEncShuffle[d];
      const int m = (int)((word >> (4 * s)) & 15u) - 8;
      sa[threadIdx.x][d] = fabsf((float)m * 0.5f);
      if (m < 0) neg |= 1u << s;
    }
    sneg[threadIdx.x] = neg;
  }
  __syncthreads();
  const int64_t i = (int64_t)blockIdx.x * ENC_THREADS + threadIdx.x;
  if (i >= n) return;
  float v[8];
  double wd[8];
  enc_load<WMODE>(x, w, scales, vps, i, v, wd);
  double best = __builtin_inf();
  uint32_t best_code = 0xFFFFFFFFu;
  for (uint32_t p = 0; p < 2; ++p) {
    const double sig = p ? -0.25 : 0.25;
    double at[8];
    uint32_t tneg = 0, freem = 0;
#pragma unroll
    for (int d = 0; d < 8; ++d) {
      const double t = (double)v[d] - sig;
      at[d] = fabs(t);
      if (t < 0.0) tneg |= 1u << kEncShuffle[d];
      if (wd[d] * at[d] == 0.0) freem |= 1u << kEncShuffle[d];
    }
    for (uint32_t r = 0; r < 256; ++r) {
      double q[8];
#pragma unroll
      for (int d = 0; d < 8; ++d) {
        const double df = at[d] - (double)sa[r][d];
        q[d] = wd[d] * (df * df);
      }
      double D = enc_tree8(q);
      const uint32_t E = tneg ^ sneg[r];  // dims to negate so that every value follows its target's sign
      uint32_t S = E ^ p;                 // stored signs (decode: eff = signs ^ parity on bit 0)
      if (freem) {
        uint32_t sf = S & ~freem;
        if ((uint32_t)(__builtin_popcount(sf) & 1) != p) sf |= freem & (0u - freem);
        S = sf;
      } else if (__builtin_popcount(E) & 1u) {
        double bd = __builtin_inf();
        uint32_t bs = 0xFFFFu;
#pragma unroll
        for (int f = 0; f < 8; ++f) {
          const double keep = q[f];
          const double df = at[f] + (double)sa[r][f];
          q[f] = wd[f] * (df * df);
          const double Df = enc_tree8(q);
          q[f] = keep;
          const uint32_t Sf = S ^ (1u << kEncShuffle[f]);
          if (Df < bd || (Df == bd && Sf < bs)) {
            bd = Df;
            bs = Sf;
          }
        }
        D = bd;
        S = bs;
      }
      const uint32_t code = (r << 8) | S;
      if (D < best || (D == best && code < best_code)) {
        best = D;
        best_code = code;
      }
    }
  }
  out[i] = (uint16_t)best_code;
}

// 8-bit E8: the 256 entries scanned in order (nibble d = dim d, value (nibble - 8) / 2).
template <int WMODE>
__global__ __launch_bounds__(ENC_THREADS) void k_e8_encode(const float* x, int64_t n, const float* w,
                                                          const uint32_t* table, const float* scales, int64_t vps,
                                                          uint8_t* out) {
#pragma clang fp contract(off)
  __shared__ float sc[256][8];
  {
    const uint32_t word = table[threadIdx.x];
#pragma unroll
    for (int d = 0; d < 8; ++d) sc[threadIdx.x][d] = (float)((int)((word >> (4 * d)) & 15u) - 8) * 0.5f;
  }
  __syncthreads();
  const int64_t i = (int64_t)blockIdx.x * ENC_THREADS + threadIdx.x;
  if (i >= n) return;
  float v[8];
  double wd[8];
  enc_load<WMODE>(x, w, scales, vps, i, v, wd);
  double best = __builtin_inf();
  uint32_t best_code = 0;
  for (uint32_t r = 0; r < 256; ++r) {
    double q[8];
#pragma unroll
    for (int d = 0; d < 8; ++d) {
      const double df = (double)v[d] - (double)sc[r][d];
      q[d] = wd[d] * (df * df);
    }
    const double D = enc_tree8(q);
    if (D < best) {  // scanned in index order: a tie keeps the lower index
      best = D;
      best_code = r;
    }
  }
  out[i] = (uint8_t)best_code;
}

// Per (row, group) max |x| / divisor in fp32 (the max_abs estimator,
// src/keep/quant/rtn.py:253-264): one wave per group.
__global__ __launch_bounds__(256) void k_group_absmax(const float* x, int64_t groups_total, int64_t group_size,
                                                      float divisor, float* scales) {
  const int64_t g = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (g >= groups_total) return;
  const float* p = x + g * group_size;
  float m = 0.f;
  for (int64_t j = lane; j < group_size; j += 64) m = fmaxf(m, fabsf(p[j]));
  for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
  if (lane == 0) scales[g] = (float)((double)m / (double)divisor);  // the correctly rounded fp32 quotient
}

template <int WMODE>
static void launch_encode(int code_bits, const float* x, int64_t n, const float* w, const uint32_t* table,
                          const float* scales, int64_t vps, void* out, hipStream_t s) {
  const dim3 grid((unsigned)((n + ENC_THREADS - 1) / ENC_THREADS)), blk(ENC_THREADS);
  if (code_bits == 16)
    hipLaunchKernelGGL((k_e8p_encode<WMODE>), grid, blk, 0, s, x, n, w, table, scales, vps, (uint16_t*)out);
  else
    hipLaunchKernelGGL((k_e8_encode<WMODE>), grid, blk, 0, s, x, n, w, table, scales, vps, (uint8_t*)out);
}

}  // namespace keep

using namespace keep;

extern "C" int keep_vq_encode(const float* vectors, int64_t n, int code_bits, const float* diagonal, int diag_mode,
                              const uint32_t* table, const float* scales, int64_t vectors_per_scale, void* codes,
                              void* stream) {
  KEEP_REQUIRE_DIMS(n, vectors_per_scale);
  KEEP_REQUIRE(code_bits == 8 || code_bits == 16, "code_bits must be 8 or 16, got %d", code_bits);
  KEEP_REQUIRE(diag_mode >= 0 && diag_mode <= 2, "diag_mode must be 0 (none), 1 (shared [8]) or 2 (per vector)");
  KEEP_REQUIRE(n >= 0, "n must be >= 0");
  if (n == 0) return KEEP_OK;
  KEEP_REQUIRE(vectors && table && codes && (diag_mode == 0 || diagonal), "null pointer argument");
  KEEP_REQUIRE(aligned(vectors, 16), "vectors must be 16-byte aligned");
  KEEP_REQUIRE(!scales || vectors_per_scale >= 1, "vectors_per_scale must be >= 1");
  KEEP_REQUIRE((n + ENC_THREADS - 1) / ENC_THREADS <= 0x7fffffffLL, "too many vectors");
  hipStream_t s = (hipStream_t)stream;
  if (diag_mode == 0) launch_encode<0>(code_bits, vectors, n, diagonal, table, scales, vectors_per_scale, codes, s);
  else if (diag_mode == 1) launch_encode<1>(code_bits, vectors, n, diagonal, table, scales, vectors_per_scale, codes, s);
  else launch_encode<2>(code_bits, vectors, n, diagonal, table, scales, vectors_per_scale, codes, s);
  return launch_status("keep_vq_encode");
}

extern "C" int keep_group_absmax(const float* x, int64_t groups_total, int64_t group_size, float divisor,
                                 float* scales, void* stream) {
  KEEP_REQUIRE_DIMS(groups_total, group_size);
  KEEP_REQUIRE(groups_total >= 0 && group_size >= 1, "bad group sizes");
  KEEP_REQUIRE(divisor > 0.f, "divisor must be positive");
  if (groups_total == 0) return KEEP_OK;
  KEEP_REQUIRE(x && scales, "null pointer argument");
  const int64_t blocks = (groups_total + 3) / 4;
  KEEP_REQUIRE(blocks <= 0x7fffffffLL, "too many groups");
  hipLaunchKernelGGL(k_group_absmax, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream, x, groups_total,
                     group_size, divisor, scales);
  return launch_status("keep_group_absmax");
}
