#pragma once
// Device helpers of the int8 matrix-core E8P kernels (moe_i8.hip, moe_tiles.hip)
// (v_mfma_i32_16x16x64_i8: exact int32 sums).
//
// Weights. Every decoded E8P weight is w = q / 4 with q an odd integer,
// |q| <= 15 (src/keep/vq/e8.py:203-234: the value v / 2 of an odd packed
// nibble v = nib - 8, negated when its effective sign bit is set, then +1/4
// for even sign parity and -1/4 for odd), so q = 2 (+-v) + sigma is exact in
// int8. Write v = 2a + 1 (a in -4..3): negating v maps a to ~a, and q = 4a' +
// 2 + sigma is the byte (a' << 2) | (2 + sigma) in two's complement. With
// T[idx] the 8 bytes 4a + 3 of the packed nibbles (no sign, even parity), a
// codeword's 8 int8 weights, in packed-nibble order, are
//   T[idx] ^ M[signs],  M[signs] byte s = (eff bit s ? 0xFC : 0) ^ (p ? 0x02 : 0),
// p the parity of the sign byte and eff = signs ^ p (bit 0 flipped when p = 1).
// That is two 8-byte lookups and a few VALU per codeword. The random lookups
// set the decode rate, so every block stages a 64 KiB image of both tables in
// LDS (built once by keep_e8p_prepare): row e (256 bytes) holds sixteen copies
// of the pair (T[e], M[e]), copy r in bytes 16 r .. 16 r + 15, and lane l reads
// copy l % 16. Sixteen consecutive lanes then touch sixteen disjoint groups of
// four banks whatever their codewords, so a lookup never waits on a bank
// conflict inside a 16-lane group. A lookup address is one byte permute:
// (idx << 8) | 16 r for T, (signs << 8) | 16 r | 8 for M.
//
// Activations. The A operand of a 16x16x64 int8 MFMA is 16 rows of 64 bytes.
// A wave's 256-element slice of the token x (fp16 or bf16) is scaled by a
// power of two s so that max |x| s lies in [32, 64), then split into int8
// terms t0 + t1 / 128 + t2 / 128^2 (each a round-to-nearest of the scaled
// remainder, so every |t| <= 64); A rows 0-2 are the three terms and the dot is
// (D0 + D1 / 128 + D2 / 128^2) / (4 s). The residual is at most 2^-20 of
// max |x| (half a unit of the last term, 1 / (2 s 128^2), with s >= 32 / max |x|).
// h (bf16) uses two terms, with the residual at most 2^-13 of its slice's max
// in base 128 (the two-launch and few-token kernels) and 2^-14 in base 256
// (the one-launch layer), so the down kernels put route r's terms in two rows
// of A. Each wave builds its terms once, in LDS.
//
// K layout. Lane l of an MFMA holds row (A) / column (B) l % 16 and 16 bytes
// of k-block l / 16. A wave's 256-wide K slice is 32 codewords; lane group g
// owns codewords 8g .. 8g + 7 (one 16-byte code load) and feeds codewords 2i,
// 2i + 1 to MFMA i, i = 0..3. A rows use the same assignment, with the eight
// values of a codeword in packed-nibble order (dims 0,2,4,6,1,3,5,7).
#include "common.h"

namespace keep {

constexpr int TQ_BYTES = 4096;     // T (256 x 8 bytes), then M (256 x 8 bytes)
constexpr int TQR_BYTES = 65536;   // the LDS image: 256 rows x 16 copies x (T, M)

typedef int q8v4 __attribute__((ext_vector_type(4)));

// B operands of one 16-byte code load (8 codewords): codewords 2i, 2i + 1 ->
// b[i], each the 8 int8 weights x 4 in packed-nibble order, T[idx] ^ M[signs]
// read from this lane's copy in the LDS image. The permutes place a
// codeword's abs index (T) or sign byte (M) in address byte 1 beside the
// lane's copy offset in byte 0 (16 r, | 8 for M). An LDS pass serves 32
// lanes, and lanes l and l + 16 share copy l % 16, so lanes of odd 16-lane
// groups look up M first and T second: within a pass one lane of a pair
// reads the copy's T half while the other reads its M half, and the XOR
// does not care about the order. lk = lookup_keys(lane) holds the two
// address bases and the four byte selectors of this lane.
struct Q8Keys {
  uint32_t base1, base2;          // copy offset for the first / second lookup
  uint32_t s1lo, s1hi, s2lo, s2hi;  // v_perm selectors (low / high codeword)
};
__device__ __forceinline__ Q8Keys q8_keys(uint32_t lane) {
  const uint32_t r16 = (lane & 15u) << 4;
  const bool m_first = (lane >> 4) & 1u;
  Q8Keys k;
  k.base1 = m_first ? (r16 | 8u) : r16;
  k.base2 = m_first ? r16 : (r16 | 8u);
  // address byte 1 <- codeword byte: T uses the abs index (bits 8-15 / 24-31),
  // M the sign byte (bits 0-7 / 16-23)
  k.s1lo = m_first ? 0x0c0c0400u : 0x0c0c0500u;
  k.s1hi = m_first ? 0x0c0c0600u : 0x0c0c0700u;
  k.s2lo = m_first ? 0x0c0c0500u : 0x0c0c0400u;
  k.s2hi = m_first ? 0x0c0c0700u : 0x0c0c0600u;
  return k;
}
// One code dword (codewords 2i, 2i + 1) -> one B operand.
__device__ __forceinline__ q8v4 q8_decode2(const char* tqr, const Q8Keys& k, uint32_t w) {
  const uint32_t a1 = __builtin_amdgcn_perm(w, k.base1, k.s1lo);
  const uint32_t a2 = __builtin_amdgcn_perm(w, k.base2, k.s2lo);
  const uint32_t b1 = __builtin_amdgcn_perm(w, k.base1, k.s1hi);
  const uint32_t b2 = __builtin_amdgcn_perm(w, k.base2, k.s2hi);
  const uint2 x1 = *(const uint2*)(tqr + a1), x2 = *(const uint2*)(tqr + a2);
  const uint2 y1 = *(const uint2*)(tqr + b1), y2 = *(const uint2*)(tqr + b2);
  return q8v4{(int)(x1.x ^ x2.x), (int)(x1.y ^ x2.y), (int)(y1.x ^ y2.x), (int)(y1.y ^ y2.y)};
}
template <bool HALVES = false>
__device__ __forceinline__ void q8_decode8(const char* tqr, const Q8Keys& k, uint4 q, q8v4 (&b)[4]) {
  const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if (HALVES && i == 2) __builtin_amdgcn_sched_barrier(0);  // at most 8 lookups in flight (register pressure)
    b[i] = q8_decode2(tqr, k, w[i]);
  }
}

// The nested tier's 8-bit E8 residual: a code byte n indexes the packed E8
// table (nibble d = dim d, value (nib - 8) / 2), so a weight x 4 is
// 2 (nib - 8), exact in int8. Its LDS image (keep_e8_1bit_prepare) holds row n
// as sixteen copies of the 8 bytes in packed-nibble order, lane l reading
// copy l % 16 (16 lanes touch disjoint bank pairs whatever their codes).
constexpr int T8R_BYTES = 32768;
__device__ __forceinline__ uint2 t8_entry(uint32_t p) {
  uint32_t b[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int d = i < 4 ? 2 * i : 2 * (i - 4) + 1;  // packed-nibble order: dims 0 2 4 6 1 3 5 7
    b[i] = (uint32_t)(2 * ((int)((p >> (4 * d)) & 15u) - 8)) & 0xffu;
  }
  return make_uint2(b[0] | b[1] << 8 | b[2] << 16 | b[3] << 24, b[4] | b[5] << 8 | b[6] << 16 | b[7] << 24);
}
// Residual code bytes w & 0xff, (w >> 8) & 0xff (codewords 2i, 2i + 1) -> one B operand.
__device__ __forceinline__ q8v4 t8_decode2(const char* img, uint32_t lane, uint32_t w) {
  const uint32_t r8 = (lane & 15u) * 8u;
  const uint2 x0 = *(const uint2*)(img + (w & 0xffu) * 128u + r8);
  const uint2 x1 = *(const uint2*)(img + ((w >> 8) & 0xffu) * 128u + r8);
  return q8v4{(int)x0.x, (int)x0.y, (int)x1.x, (int)x1.y};
}

__device__ __forceinline__ q8v4 mfma_i8(q8v4 a, q8v4 b, q8v4 c) {
  return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
}

// Power-of-two s with max_abs * s in [32, 64) (max_abs > 0), and 1 / (4 s);
// NaN for a non-finite max_abs, so that it reaches the outputs.
__device__ __forceinline__ void q8_scale(float max_abs, float& s, float& inv4s) {
  const int e = max_abs > 0.f ? (int)((__float_as_uint(max_abs) >> 23) & 0xffu) - 126 : 0;  // max_abs < 2^e
  const int es = min(max(127 + 6 - e, 1), 254), ei = min(max(127 - 8 + e, 1), 254);
  s = __uint_as_float((uint32_t)es << 23);
  inv4s = max_abs < __builtin_inff() ? __uint_as_float((uint32_t)ei << 23) : __builtin_nanf("");
}

__device__ __forceinline__ uint32_t q8_pack4(float a, float b, float c, float d) {
  return ((uint32_t)(int)a & 0xffu) | (((uint32_t)(int)b & 0xffu) << 8) | (((uint32_t)(int)c & 0xffu) << 16) |
         ((uint32_t)(int)d << 24);
}

// The four values of this lane in a 16-byte chunk of 8 fp16 / bf16 values:
// dims 2t + half, t = 0..3 (packed-nibble positions 4 half + t).
template <bool BF>
__device__ __forceinline__ void q8_half4(uint4 c, uint32_t half, float (&v)[4]) {
  const uint32_t w[4] = {c.x, c.y, c.z, c.w};
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const uint32_t hb = half ? (w[t] >> 16) : (w[t] & 0xffffu);
    if constexpr (BF) v[t] = __uint_as_float(hb << 16);
    else v[t] = (float)__builtin_bit_cast(_Float16, (uint16_t)hb);
  }
}

// NTERM int8 terms of the four values v x s, packed four to a word.
template <int NTERM>
__device__ __forceinline__ void q8_terms(const float (&v)[4], float s, uint32_t (&out)[NTERM]) {
  float y[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) y[t] = v[t] * s;
#pragma unroll
  for (int n = 0; n < NTERM; ++n) {
    float r[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      r[t] = rintf(y[t]);
      y[t] = (y[t] - r[t]) * 128.f;
    }
    out[n] = q8_pack4(r[0], r[1], r[2], r[3]);
  }
}

// The two int8 terms t0 + t1 / 128 = rint(v s 128) / 128 of four values
// (|v| s < 64), the sum q8_terms<2> represents: the FMA with 1.5 * 2^23
// leaves rint(v s 128) in the low 16 bits of the result (two's complement,
// |.| < 2^13), and the digits t0 = (F + 64) >> 7, t1 = ((F + 64) & 127) - 64
// are formed two values at a time in 16-bit halves.
__device__ __forceinline__ void q8_digits2(const float (&v)[4], float s, uint32_t (&out)[2]) {
  typedef short s16x2 __attribute__((ext_vector_type(2)));
  const float s128 = s * 128.f;
  uint32_t f[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) f[t] = __float_as_uint(fmaf(v[t], s128, 12582912.0f));
  const s16x2 g01 = __builtin_bit_cast(s16x2, __builtin_amdgcn_perm(f[1], f[0], 0x05040100u)) + (short)64;
  const s16x2 g23 = __builtin_bit_cast(s16x2, __builtin_amdgcn_perm(f[3], f[2], 0x05040100u)) + (short)64;
  const s16x2 h01 = g01 >> (short)7, h23 = g23 >> (short)7;
  const s16x2 l01 = (g01 & (short)127) - (short)64, l23 = (g23 & (short)127) - (short)64;
  // the low byte of each half, values 0..3 in bytes 0..3
  out[0] = __builtin_amdgcn_perm(__builtin_bit_cast(uint32_t, h23), __builtin_bit_cast(uint32_t, h01), 0x06040200u);
  out[1] = __builtin_amdgcn_perm(__builtin_bit_cast(uint32_t, l23), __builtin_bit_cast(uint32_t, l01), 0x06040200u);
}

// The same two terms in base 256, t0 + t1 / 256 = rint(v s 256) / 256 of four
// values (|v| s < 64), from s256 = s * 256 (a power of two): the FMA with
// 1.5 * 2^23 + 128 leaves F + 128 = rint(v s 256) + 128 in the low 16 bits of
// the float (two's complement); t0 is its high byte, floor((F + 128) / 256)
// (|t0| <= 64), and t1 = F - 256 t0 is its low byte minus 128, i.e. the low
// byte with bit 7 flipped. Four FMAs, four byte permutes and one XOR.
__device__ __forceinline__ void q8_digits2_b256(const float (&v)[4], float s256, uint32_t (&out)[2]) {
  uint32_t f[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) f[t] = __float_as_uint(fmaf(v[t], s256, 12583040.0f));
  const uint32_t p01 = __builtin_amdgcn_perm(f[1], f[0], 0x05040100u);  // F + 128 of values 0, 1
  const uint32_t p23 = __builtin_amdgcn_perm(f[3], f[2], 0x05040100u);  // of values 2, 3
  out[0] = __builtin_amdgcn_perm(p23, p01, 0x07050301u);                // high bytes
  out[1] = __builtin_amdgcn_perm(p23, p01, 0x06040200u) ^ 0x80808080u;  // low bytes - 128
}

// Word index in an A-term buffer of 16-byte slots [row][g * 4 + i] for the
// lane writing chunk c (0..31 of the wave's slice), half `half`.
__device__ __forceinline__ uint32_t q8_aword(uint32_t row, uint32_t c, uint32_t half) {
  return (row * 16u + (c >> 3) * 4u + ((c & 7u) >> 1)) * 4u + (c & 1u) * 2u + half;
}

__device__ __forceinline__ uint4 ldg16_q(const void* p) {
  typedef unsigned int v4u __attribute__((ext_vector_type(4)));
  const v4u v = *(const __attribute__((address_space(1))) v4u*)p;
  return uint4{v.x, v.y, v.z, v.w};
}

__device__ __forceinline__ uint32_t ldg4_q(const void* p) { return *(const __attribute__((address_space(1))) uint32_t*)p; }

__device__ __forceinline__ uint2 ldg8_q(const void* p) {
  typedef unsigned int v2u __attribute__((ext_vector_type(2)));
  const v2u v = *(const __attribute__((address_space(1))) v2u*)p;
  return make_uint2(v.x, v.y);
}

// 4-byte LDS DMA: the active lanes' words land at lds_wave_base + 4 * lane.
__device__ __forceinline__ void dma4_q(const void* g, uint32_t* lds_wave_base) {
  __builtin_amdgcn_global_load_lds(g, (__attribute__((address_space(3))) void*)lds_wave_base, 4, 0, 0);
}

__device__ __forceinline__ void dma16_q(const uint4* g, uint4* lds_wave_base) {
  __builtin_amdgcn_global_load_lds((const void*)g, (__attribute__((address_space(3))) void*)lds_wave_base, 16, 0,
                                   0);
}

template <int N>
__device__ __forceinline__ void wait_vm_q() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// Offsets in the prepared buffer (keep_e8p_prepare): T and M, then the flag
// word, then the 64 KiB LDS image.
constexpr size_t TQ_OFFSET = 0;
constexpr size_t TQ_FLAG_OFFSET = TQ_OFFSET + TQ_BYTES;
constexpr size_t TQR_OFFSET = TQ_FLAG_OFFSET + 256u;

}  // namespace keep
