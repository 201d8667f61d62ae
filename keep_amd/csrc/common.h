// Shared device helpers for the gfx950 routed E8P kernels.
//
// E8P codeword c (uint16): bits 0-7 are signs, bits 8-15 index the 256-entry
// packed abs table (nibble j of an entry = value*2 + 8). Output dim d reads
// nibble {0,4,1,5,2,6,3,7}[d], so dims (2k, 2k+1) are nibbles (k, k+4) and are
// held as one packed 16-bit pair. With p = popcount(signs) & 1 and
// eff = signs ^ p, nibble s is negated when bit s of eff is set, and every
// value gets +1/4 (p = 0) or -1/4 (p = 1) -- the reference decoder
// src/keep/vq/e8.py:203-234 restated. Every decoded value is k/4, |k| <= 15,
// exact in fp16 and bf16.
//
// LDS codebook entry (uint4): word k = pair (dim 2k | dim 2k+1 << 16) of the
// *unsigned-by-codeword* values, in fp16 or bf16 bits. Signs are applied by
// XOR of bit 15 / bit 31 and the +-1/4 shift as +-0.25 * sum(x of the 8 dims)
// (the form of src/ramp/kernels/e8p_m1.metal:81-92), which is exact algebra.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <initializer_list>

#include "../../include/keep_amd.h"

namespace keep {

typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
typedef __bf16 b2_t __attribute__((ext_vector_type(2)));

// ---------------------------------------------------------------- host-side errors
void set_error(const char* fmt, ...);
int launch_status(const char* what);

#define KEEP_REQUIRE(cond, ...)          \
  do {                                   \
    if (!(cond)) {                       \
      ::keep::set_error(__VA_ARGS__);    \
      return KEEP_EINVAL;                \
    }                                    \
  } while (0)

inline bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }
inline int dtype_size(int dt) { return dt == KEEP_F32 ? 4 : 2; }
inline bool dtype_ok(int dt) { return dt == KEEP_F32 || dt == KEEP_F16 || dt == KEEP_BF16; }
// Every size an entry point takes lies in [0, 2^31) (the kernels index in 32
// bits). Checked first, so that the products later checks form (two sizes, or
// a size and a small constant) cannot overflow int64.
constexpr int64_t KEEP_DIM_LIMIT = int64_t(1) << 31;
inline bool dims_ok(std::initializer_list<int64_t> dims) {
  for (int64_t d : dims)
    if (d < 0 || d >= KEEP_DIM_LIMIT) return false;
  return true;
}
#define KEEP_REQUIRE_DIMS(...) KEEP_REQUIRE(::keep::dims_ok({__VA_ARGS__}), "every size must be in [0, 2^31)")

// ---------------------------------------------------------------- element types
struct bf16s {
  uint16_t bits;
};

__device__ __forceinline__ float to_float(float v) { return v; }
__device__ __forceinline__ float to_float(_Float16 v) { return (float)v; }
__device__ __forceinline__ float to_float(bf16s v) { return __uint_as_float((uint32_t)v.bits << 16); }

template <typename T>
__device__ __forceinline__ T from_float(float v);
template <>
__device__ __forceinline__ float from_float<float>(float v) { return v; }
template <>
__device__ __forceinline__ _Float16 from_float<_Float16>(float v) { return (_Float16)v; }
template <>
__device__ __forceinline__ bf16s from_float<bf16s>(float v) {
  // round to nearest even; NaN stays NaN
  uint32_t u = __float_as_uint(v);
  if ((u & 0x7fffffffu) > 0x7f800000u) return bf16s{(uint16_t)((u >> 16) | 0x40u)};
  u += 0x7fffu + ((u >> 16) & 1u);
  return bf16s{(uint16_t)(u >> 16)};
}

// Packed pair element kind used in the LDS codebook and for activations.
enum PairKind { PAIR_F16 = 0, PAIR_BF16 = 1 };

template <int PK>
__device__ __forceinline__ uint32_t encode_half_units(int v2) {
  // v2 = value * 2 (an odd or even small integer); returns 16-bit pattern of v2/2
  float f = (float)v2 * 0.5f;
  if constexpr (PK == PAIR_F16) {
    _Float16 h = (_Float16)f;
    return (uint32_t)__builtin_bit_cast(uint16_t, h);
  } else {
    return __float_as_uint(f) >> 16;  // exact: at most 4 significant bits
  }
}

template <int PK>
__device__ __forceinline__ float dot2(uint32_t w, uint32_t x, float acc) {
  if constexpr (PK == PAIR_F16) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(h2_t, w), __builtin_bit_cast(h2_t, x), acc, false);
  } else {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(b2_t, w), __builtin_bit_cast(b2_t, x), acc, false);
  }
}

template <int PK>
__device__ __forceinline__ float pair_lo(uint32_t w) {
  if constexpr (PK == PAIR_F16) return (float)__builtin_bit_cast(_Float16, (uint16_t)(w & 0xffffu));
  else return __uint_as_float(w << 16);
}
template <int PK>
__device__ __forceinline__ float pair_hi(uint32_t w) {
  if constexpr (PK == PAIR_F16) return (float)__builtin_bit_cast(_Float16, (uint16_t)(w >> 16));
  else return __uint_as_float(w & 0xffff0000u);
}

// Build the LDS codebook from a packed nibble table (block-cooperative).
// CB = 16: E8P abs table, pair k = nibbles (k, k+4). CB = 8: E8 table,
// pair k = nibbles (2k, 2k+1) (dim d = nibble d).
template <int CB, int PK>
__device__ __forceinline__ void codebook_entry(uint4* tab, int i, uint32_t p) {
  uint32_t w[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int lo_n = CB == 16 ? k : 2 * k;
    const int hi_n = CB == 16 ? k + 4 : 2 * k + 1;
    const int lo = (int)((p >> (4 * lo_n)) & 15u) - 8;
    const int hi = (int)((p >> (4 * hi_n)) & 15u) - 8;
    w[k] = encode_half_units<PK>(lo) | (encode_half_units<PK>(hi) << 16);
  }
  tab[i] = make_uint4(w[0], w[1], w[2], w[3]);
}
template <int CB, int PK>
__device__ __forceinline__ void build_codebook(uint4* tab, const uint32_t* packed) {
  for (int i = threadIdx.x; i < 256; i += blockDim.x) codebook_entry<CB, PK>(tab, i, packed[i]);
}

// Residual table given as fp16 half2 pairs uint32[256*4]; converted to PK.
template <int PK>
__device__ __forceinline__ void load_pair_table(uint4* tab, const uint32_t* pairs) {
  for (int i = threadIdx.x; i < 256; i += blockDim.x) {
    uint32_t w[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      uint32_t v = pairs[4 * i + k];
      if constexpr (PK == PAIR_BF16) {
        float lo = (float)__builtin_bit_cast(_Float16, (uint16_t)(v & 0xffffu));
        float hi = (float)__builtin_bit_cast(_Float16, (uint16_t)(v >> 16));
        v = (__float_as_uint(lo) >> 16) | (__float_as_uint(hi) & 0xffff0000u);
      }
      w[k] = v;
    }
    tab[i] = make_uint4(w[0], w[1], w[2], w[3]);
  }
}

// Signs of one E8P codeword as XOR masks on the four pairs, plus the shift.
struct E8PSigns {
  uint32_t m0, m1, m2, m3;
  float shift;  // +0.25 or -0.25
};

__device__ __forceinline__ E8PSigns e8p_signs(uint32_t c) {
  const uint32_t s = c & 0xffu;
  const uint32_t p = __builtin_popcount(s) & 1u;
  const uint32_t eff = s ^ p;
  // bit k -> bit k, bit k+4 -> bit k+16; pair k then needs bits (k, k+16) at (15, 31)
  const uint32_t sp = (eff & 0x0fu) | ((eff & 0xf0u) << 12);
  E8PSigns r;
  r.m0 = (sp << 15) & 0x80008000u;
  r.m1 = (sp << 14) & 0x80008000u;
  r.m2 = (sp << 13) & 0x80008000u;
  r.m3 = (sp << 12) & 0x80008000u;
  r.shift = p ? -0.25f : 0.25f;
  return r;
}

// acc + <decode(c), x> for one E8P codeword; xv = 4 packed activation pairs,
// xs = sum of the 8 activations (fp32).
template <int PK>
__device__ __forceinline__ float e8p_dot(uint32_t c, const uint4* tab, const uint32_t* xv, float xs, float acc) {
  const E8PSigns sg = e8p_signs(c);
  const uint4 e = tab[(c >> 8) & 0xffu];
  acc = dot2<PK>(e.x ^ sg.m0, xv[0], acc);
  acc = dot2<PK>(e.y ^ sg.m1, xv[1], acc);
  acc = dot2<PK>(e.z ^ sg.m2, xv[2], acc);
  acc = dot2<PK>(e.w ^ sg.m3, xv[3], acc);
  return fmaf(sg.shift, xs, acc);
}

// fp32 activations: decode pairs to float and FMA.
__device__ __forceinline__ float e8p_dot_f32(uint32_t c, const uint4* tab, const float* xf, float xs, float acc) {
  const E8PSigns sg = e8p_signs(c);
  const uint4 e = tab[(c >> 8) & 0xffu];
  const uint32_t w0 = e.x ^ sg.m0, w1 = e.y ^ sg.m1, w2 = e.z ^ sg.m2, w3 = e.w ^ sg.m3;
  acc = fmaf(pair_lo<PAIR_F16>(w0), xf[0], acc);
  acc = fmaf(pair_hi<PAIR_F16>(w0), xf[1], acc);
  acc = fmaf(pair_lo<PAIR_F16>(w1), xf[2], acc);
  acc = fmaf(pair_hi<PAIR_F16>(w1), xf[3], acc);
  acc = fmaf(pair_lo<PAIR_F16>(w2), xf[4], acc);
  acc = fmaf(pair_hi<PAIR_F16>(w2), xf[5], acc);
  acc = fmaf(pair_lo<PAIR_F16>(w3), xf[6], acc);
  acc = fmaf(pair_hi<PAIR_F16>(w3), xf[7], acc);
  return fmaf(sg.shift, xs, acc);
}

// 8-bit E8 codeword: a signed table row, no sign bits, no shift.
template <int PK>
__device__ __forceinline__ float e8_dot(uint32_t c, const uint4* tab, const uint32_t* xv, float acc) {
  const uint4 e = tab[c & 0xffu];
  acc = dot2<PK>(e.x, xv[0], acc);
  acc = dot2<PK>(e.y, xv[1], acc);
  acc = dot2<PK>(e.z, xv[2], acc);
  acc = dot2<PK>(e.w, xv[3], acc);
  return acc;
}

__device__ __forceinline__ float e8_dot_f32(uint32_t c, const uint4* tab, const float* xf, float acc) {
  const uint4 e = tab[c & 0xffu];
  acc = fmaf(pair_lo<PAIR_F16>(e.x), xf[0], acc);
  acc = fmaf(pair_hi<PAIR_F16>(e.x), xf[1], acc);
  acc = fmaf(pair_lo<PAIR_F16>(e.y), xf[2], acc);
  acc = fmaf(pair_hi<PAIR_F16>(e.y), xf[3], acc);
  acc = fmaf(pair_lo<PAIR_F16>(e.z), xf[4], acc);
  acc = fmaf(pair_hi<PAIR_F16>(e.z), xf[5], acc);
  acc = fmaf(pair_lo<PAIR_F16>(e.w), xf[6], acc);
  acc = fmaf(pair_hi<PAIR_F16>(e.w), xf[7], acc);
  return acc;
}

// Deterministic wave64 butterfly sum; every lane ends with the total.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m, 64));
  return v;
}

// Codes chunk of CH codewords (CB-bit) starting at codeword index `cw` of a row.
template <int CB, int CH>
__device__ __forceinline__ void load_codes(const void* row_base, int64_t cw, uint32_t* words) {
  constexpr int BYTES = CH * CB / 8;
  const char* p = (const char*)row_base + cw * (CB / 8);
  if constexpr (BYTES == 16) {
    uint4 v = *(const uint4*)p;
    words[0] = v.x; words[1] = v.y; words[2] = v.z; words[3] = v.w;
  } else if constexpr (BYTES == 8) {
    uint2 v = *(const uint2*)p;
    words[0] = v.x; words[1] = v.y;
  } else if constexpr (BYTES == 4) {
    words[0] = *(const uint32_t*)p;
  } else if constexpr (BYTES == 2) {
    words[0] = *(const uint16_t*)p;
  } else {
    words[0] = *(const uint8_t*)p;
  }
}

template <int CB>
__device__ __forceinline__ uint32_t codeword_at(const uint32_t* words, int i) {
  if constexpr (CB == 16) return (words[i >> 1] >> ((i & 1) * 16)) & 0xffffu;
  else return (words[i >> 2] >> ((i & 3) * 8)) & 0xffu;
}

// Activation chunk: CH codewords = CH*8 values starting at element 8*cw.
// 16-bit activations are kept as packed pairs; sums in fp32.
template <typename XT, int CH>
struct XChunk {
  uint32_t v[CH * 4];
  float s[CH];
  __device__ __forceinline__ void load(const XT* xrow, int64_t cw) {
    const uint4* p = (const uint4*)(xrow + cw * 8);
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      uint4 q = p[i];
      v[4 * i + 0] = q.x; v[4 * i + 1] = q.y; v[4 * i + 2] = q.z; v[4 * i + 3] = q.w;
      float t = 0.f;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        uint32_t w = v[4 * i + k];
        if constexpr (sizeof(XT) == 2 && !__is_same(XT, bf16s)) {
          t += pair_lo<PAIR_F16>(w) + pair_hi<PAIR_F16>(w);
        } else {
          t += pair_lo<PAIR_BF16>(w) + pair_hi<PAIR_BF16>(w);
        }
      }
      s[i] = t;
    }
  }
};

template <int CH>
struct XChunk<float, CH> {
  float v[CH * 8];
  float s[CH];
  __device__ __forceinline__ void load(const float* xrow, int64_t cw) {
    const float4* p = (const float4*)(xrow + cw * 8);
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      float4 a = p[2 * i], b = p[2 * i + 1];
      v[8 * i + 0] = a.x; v[8 * i + 1] = a.y; v[8 * i + 2] = a.z; v[8 * i + 3] = a.w;
      v[8 * i + 4] = b.x; v[8 * i + 5] = b.y; v[8 * i + 6] = b.z; v[8 * i + 7] = b.w;
      s[i] = ((a.x + a.y) + (a.z + a.w)) + ((b.x + b.y) + (b.z + b.w));
    }
  }
};

template <typename XT>
struct PairOf {
  static constexpr int value = PAIR_F16;
};
template <>
struct PairOf<bf16s> {
  static constexpr int value = PAIR_BF16;
};

// Partial dot of one row chunk (CH codewords) with an activation chunk.
template <int CB, typename XT, int CH>
__device__ __forceinline__ float chunk_dot(const uint32_t* words, const uint4* tab, const XChunk<XT, CH>& xc) {
  constexpr int PK = PairOf<XT>::value;
  float part = 0.f;
#pragma unroll
  for (int i = 0; i < CH; ++i) {
    const uint32_t c = codeword_at<CB>(words, i);
    if constexpr (__is_same(XT, float)) {
      if constexpr (CB == 16) part = e8p_dot_f32(c, tab, xc.v + 8 * i, xc.s[i], part);
      else part = e8_dot_f32(c, tab, xc.v + 8 * i, part);
    } else {
      if constexpr (CB == 16) part = e8p_dot<PK>(c, tab, xc.v + 4 * i, xc.s[i], part);
      else part = e8_dot<PK>(c, tab, xc.v + 4 * i, part);
    }
  }
  return part;
}

template <typename ST>
__device__ __forceinline__ float load_scale(const void* scales, int64_t i) {
  return to_float(((const ST*)scales)[i]);
}

}  // namespace keep
