// Fused routed SwiGLU MoE decode for gfx950 with the expanded E8P table.
//
// Per codeword the decode is two LDS lookups and four v_dot2: the signs,
// the parity bit and the +-1/4 shift of E8P (src/keep/vq/e8.py:203-234) are
// folded into a 128 KiB table so no sign arithmetic runs per codeword.
//
// Expanded table (built once per codebook by keep_e8p_prepare): 16384
// entries of 8 bytes (four packed fp16 or bf16 values). Byte address
//     (p << 16) | (half << 15) | (idx << 7) | (nibble << 3)
// with p = popcount(signs) & 1, idx = c >> 8 and
//   half 0 ("H"): nibble = sign bits 4-7; values of dims 1,3,5,7
//                 (packed nibbles 4-7), signed by sign bits 4-7;
//   half 1 ("L"): nibble = sign bits 0-3; values of dims 0,2,4,6
//                 (packed nibbles 0-3), signed by bits 0-3 with bit 0 ^ p;
// every value + 1/4 (p = 0) or - 1/4 (p = 1). So an H entry is
// (d1, d3 | d5, d7) and an L entry (d0, d2 | d4, d6), and activations are
// paired the same way: (x0,x2) (x4,x6) (x1,x3) (x5,x7).
//
// Kernels run one 1024-thread block per CU (the table takes 128 KiB of its
// 160 KiB LDS). Every wave first issues the global loads of the table copy,
// then all of its code, activation and scale loads, and only then writes the
// table to LDS and joins the barrier, so the HBM stream is in flight while
// the table is staged. Lane reductions use DPP row ops plus readlane.
#include <mutex>

#include "common.h"
#include "moe_dev.h"
#include "route_dev.h"

namespace keep {

constexpr int XT_ENTRIES = 16384;                 // 8-byte entries
constexpr int XT_BYTES = XT_ENTRIES * 8;          // 128 KiB
constexpr int MOE_THREADS = 1024;
constexpr int MOE_WAVES = MOE_THREADS / 64;

// ------------------------------------------------------------------ expanded table

template <int PK>
__global__ __launch_bounds__(256) void k_expand_table(const uint32_t* packed, uint2* out) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= XT_ENTRIES) return;
  const int p = (i >> 13) & 1;
  const int half = (i >> 12) & 1;
  const int idx = (i >> 4) & 255;
  const int nib = i & 15;
  const uint32_t word = packed[idx];
  const float shift = p ? -0.25f : 0.25f;
  uint32_t h[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int n = half ? j : 4 + j;  // packed nibble
    int sbit = (nib >> j) & 1;
    if (half && j == 0) sbit ^= p;
    float v = (float)((int)((word >> (4 * n)) & 15u) - 8) * 0.5f;
    if (sbit) v = -v;
    v += shift;
    if constexpr (PK == PAIR_F16) h[j] = (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)v);
    else h[j] = __float_as_uint(v) >> 16;  // exact (at most 4 significant bits)
  }
  out[i] = make_uint2(h[0] | (h[1] << 16), h[2] | (h[3] << 16));
}

// ------------------------------------------------------------------ device helpers

__device__ __forceinline__ float dpp_row_sum(float v) {
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x141, 0xF, 0xF, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x140, 0xF, 0xF, false));
  return v;  // every lane of each 16-lane row holds its row's sum
}

// Wave-uniform total of v over 64 lanes (fixed order).
__device__ __forceinline__ float wave_total(float v) {
  v = dpp_row_sum(v);
  const float a = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0));
  const float b = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 16));
  const float c = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 32));
  const float d = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 48));
  return (a + b) + (c + d);
}

// LDS byte addresses of the H and L entries of the codeword in bits
// [lo, lo + 16) of w (lo = 0 or 16).
template <int LO>
__device__ __forceinline__ void xt_addr(uint32_t w, uint32_t& ah, uint32_t& al) {
  const uint32_t hb = __builtin_amdgcn_ubfe(w, LO + 4, 12);  // idx << 4 | sign bits 4-7
  const uint32_t pc = __builtin_popcount(__builtin_amdgcn_ubfe(w, LO, 8));
  ah = ((hb << 3)) | ((pc << 16) & 0x10000u);
  const uint32_t lo_nib = LO ? (w >> 13) : (w << 3);  // sign bits 0-3 at bits 3-6
  al = (ah & ~0x78u) | (lo_nib & 0x78u);
}

template <int PK>
__device__ __forceinline__ float xt_dot(const char* tab, uint32_t ah, uint32_t al, const uint32_t* xp, float acc) {
  const uint2 eh = *(const uint2*)(tab + ah);
  const uint2 el = *(const uint2*)(tab + al + 0x8000);
  acc = dot2<PK>(el.x, xp[0], acc);
  acc = dot2<PK>(el.y, xp[1], acc);
  acc = dot2<PK>(eh.x, xp[2], acc);
  acc = dot2<PK>(eh.y, xp[3], acc);
  return acc;
}

// Natural activation pairs (x0,x1)(x2,x3)(x4,x5)(x6,x7) -> table order
// (x0,x2)(x4,x6)(x1,x3)(x5,x7).
__device__ __forceinline__ void permute_x(const uint4 q, uint32_t* xp) {
  xp[0] = __builtin_amdgcn_perm(q.y, q.x, 0x05040100u);
  xp[1] = __builtin_amdgcn_perm(q.w, q.z, 0x05040100u);
  xp[2] = __builtin_amdgcn_perm(q.y, q.x, 0x07060302u);
  xp[3] = __builtin_amdgcn_perm(q.w, q.z, 0x07060302u);
}

__device__ __forceinline__ float scale_of(const void* p, int dt, int64_t i) {
  if (dt == KEEP_F16) return (float)((const _Float16*)p)[i];
  if (dt == KEEP_BF16) return __uint_as_float((uint32_t)((const uint16_t*)p)[i] << 16);
  return ((const float*)p)[i];
}

struct MoeV2Args {
  const void* x;  // [T, H] fp16/bf16
  int32_t T, H, I, k, E;
  const int32_t* idx;
  const float* w;
  const uint16_t *gc, *uc, *dc;
  const void *gs, *us, *ds;
  int sdt;
  int32_t Gh, cpg_h, Gi, cpg_i;
  const uint4* xt_x;  // expanded table in the activation pair kind
  const uint4* xt_h;  // expanded table in bf16 (for h)
  float limit;
  uint16_t* h;  // [T, k, I] bf16, natural order (the layout every MoE path shares)
  void* out;
  int odt;
  int32_t units, rows_per_token;
};

typedef __attribute__((address_space(3))) void* lds_ptr_t;

// Stream 1 KiB (64 lanes x 16 B) from global memory straight into LDS.
__device__ __forceinline__ void dma16(const uint4* g, uint4* lds_wave_base) {
  __builtin_amdgcn_global_load_lds((const void*)g, (lds_ptr_t)lds_wave_base, 16, 0, 0);
}

// Wait until at most n vector-memory operations of this wave are outstanding
// (gfx9 s_waitcnt encoding; expcnt and lgkmcnt left at their maxima).
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// Each wave streams its 1/16 of the 128 KiB table.
__device__ __forceinline__ void table_dma(const uint4* g, uint4* tab4, int wv, int lane) {
#pragma unroll
  for (int i = 0; i < XT_BYTES / 16 / MOE_THREADS; ++i)
    dma16(g + i * MOE_THREADS + wv * 64 + lane, tab4 + i * MOE_THREADS + wv * 64);
}

template <int CH>
__device__ __forceinline__ void load_cw(const uint16_t* p, uint32_t* w) {
  if constexpr (CH == 8) {
    const uint4 q = *(const uint4*)p;
    w[0] = q.x; w[1] = q.y; w[2] = q.z; w[3] = q.w;
  } else if constexpr (CH == 4) {
    const uint2 q = *(const uint2*)p;
    w[0] = q.x; w[1] = q.y;
  } else {
    w[0] = *(const uint32_t*)p;
  }
}


// ------------------------------------------------------------------ gate/up/SwiGLU

// A unit is R consecutive rows of the flattened [T, k, I] row space; a block
// (NWAV units) never straddles a token (NWAV * R divides k * I). A wave
// computes gate and up for its R rows and writes h = SwiGLU(gate, up) in
// bf16, table order. Lanes split K: CH codewords per lane per step, STEPS
// steps. Route metadata is read with scalar loads before the LDS DMA group so
// the barrier waits only on the DMA, never on the code stream.
template <int PK, int NWAV, int R, int CH, int STEPS>
__global__ __launch_bounds__(NWAV * 64) void k_moe_gateup_v2(MoeV2Args a) {
  __shared__ uint4 tab4[XT_BYTES / 16];
  __shared__ uint4 xsh[1024];  // the block's token row, natural order (H <= 8192)
  const char* tab = (const char*)tab4;
  constexpr int NW = CH / 2;
  constexpr int NLOADS = 2 * R * STEPS;  // code loads per lane, issued after the DMA group
  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t C = (uint32_t)a.H >> 3;

  // 0. route metadata (scalar)
  const uint32_t unit = blockIdx.x * NWAV + wv;
  const bool active = unit < (uint32_t)a.units;
  const uint32_t rf0 = (active ? unit : 0) * R;
  uint32_t route = rf0 / (uint32_t)a.I;
  uint32_t row = rf0 - route * (uint32_t)a.I;
  uint32_t base[R];
  bool rok[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    if (r > 0 && ++row == (uint32_t)a.I) {
      row = 0;
      ++route;
    }
    const int32_t e = a.idx[route];
    rok[r] = active && e >= 0 && e < a.E && a.w[route] != 0.f;
    base[r] = rok[r] ? (uint32_t)e * a.I + row : 0u;
  }

  // 1. LDS DMA: table and the token row
#pragma unroll
  for (int i = 0; i < XT_BYTES / 16 / (NWAV * 64); ++i)
    dma16(a.xt_x + i * NWAV * 64 + wv * 64 + lane, tab4 + i * NWAV * 64 + wv * 64);
  const uint32_t t = ((uint32_t)blockIdx.x * NWAV * R) / (uint32_t)a.rows_per_token;
  const uint4* xg = (const uint4*)((const uint16_t*)a.x + (size_t)t * a.H);
  for (uint32_t c0 = wv * 64; c0 < C; c0 += NWAV * 64) {
    const uint32_t c = c0 + lane < C ? c0 + lane : C - 1;
    dma16(xg + c, xsh + c0);
  }
  __builtin_amdgcn_sched_barrier(0);

  // 2. codes and scales of this wave's unit (exactly NLOADS vector loads)
  uint32_t gw[R][STEPS][NW], uw[R][STEPS][NW];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const uint16_t* grow = a.gc + (size_t)base[r] * C;
    const uint16_t* urow = a.uc + (size_t)base[r] * C;
#pragma unroll
    for (int s = 0; s < STEPS; ++s) {
      uint32_t cw = lane * CH + s * 64 * CH;
      cw = cw < C ? cw : 0u;
      load_cw<CH>(grow + cw, gw[r][s]);
      load_cw<CH>(urow + cw, uw[r][s]);
    }
  }
  __builtin_amdgcn_sched_barrier(0);
  wait_vm<NLOADS>();  // DMA group complete; codes may still be in flight
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_sched_barrier(0);
  if (!active) return;
  // scales: consumed when a row's dot is done, so their latency hides behind the decode
  ScaleRaw gsr[R][STEPS], usr[R][STEPS];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int s = 0; s < STEPS; ++s) {
      uint32_t cw = lane * CH + s * 64 * CH;
      cw = cw < C ? cw : 0u;
      const uint32_t si = base[r] * a.Gh + cw / a.cpg_h;
      gsr[r][s] = scale_raw(a.gs, a.sdt, si);
      usr[r][s] = scale_raw(a.us, a.sdt, si);
    }

  float ag[R], au[R];
#pragma unroll
  for (int r = 0; r < R; ++r) ag[r] = au[r] = 0.f;
#pragma unroll
  for (int s = 0; s < STEPS; ++s) {
    const uint32_t cw0 = lane * CH + s * 64 * CH;
    float pg[R], pu[R];
#pragma unroll
    for (int r = 0; r < R; ++r) pg[r] = pu[r] = 0.f;
    // codeword-outer, row-inner: one activation chunk live, shared by all 2R rows
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      uint32_t xp[4];
      permute_x(xsh[cw0 + i < C ? cw0 + i : 0], xp);
#pragma unroll
      for (int r = 0; r < R; ++r) {
        uint32_t ah, al;
        if (i & 1) xt_addr<16>(gw[r][s][i >> 1], ah, al);
        else xt_addr<0>(gw[r][s][i >> 1], ah, al);
        pg[r] = xt_dot<PK>(tab, ah, al, xp, pg[r]);
        if (i & 1) xt_addr<16>(uw[r][s][i >> 1], ah, al);
        else xt_addr<0>(uw[r][s][i >> 1], ah, al);
        pu[r] = xt_dot<PK>(tab, ah, al, xp, pu[r]);
      }
      // keep the address math and lookups of later codewords out of this one
      asm volatile("" ::: "memory");
      __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const float keep = (rok[r] && cw0 < C) ? 1.f : 0.f;
      const uint32_t si = base[r] * a.Gh + (cw0 < C ? cw0 : 0u) / a.cpg_h;
      ag[r] = fmaf(pg[r], keep * scale_cvt(gsr[r][s], a.sdt, si), ag[r]);
      au[r] = fmaf(pu[r], keep * scale_cvt(usr[r][s], a.sdt, si), au[r]);
    }
  }
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const float g = wave_total(ag[r]);
    const float u = wave_total(au[r]);
    if (lane == r && rok[r]) {
      const uint32_t rf = rf0 + r;
      a.h[rf] = from_float<bf16s>(silu_mul(g, u, a.limit)).bits;
    }
  }
}

// ------------------------------------------------------------------ down + combine

// A block serves one token and MOE_WAVES * R output rows; the token's h
// (k * I bf16 in table order) is streamed into LDS. A wave computes R output
// rows over all k routes with the weighted fp32 sum.
template <int R, int CH, int STEPS, int KMAX>
__global__ __launch_bounds__(MOE_THREADS) void k_moe_down_v2(MoeV2Args a) {
  __shared__ uint4 tab4[XT_BYTES / 16];
  __shared__ uint4 hsh[1536];  // k * I / 8 <= 1536 codewords (24 KiB)
  const char* tab = (const char*)tab4;
  constexpr int NW = CH / 2;
  constexpr int NLOADS = KMAX * R * STEPS;
  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t bpt = ((uint32_t)a.H + MOE_WAVES * R - 1) / (MOE_WAVES * R);
  const uint32_t t = blockIdx.x / bpt;
  const uint32_t row0 = (blockIdx.x - t * bpt) * (MOE_WAVES * R) + wv * R;
  const uint32_t C = (uint32_t)a.I >> 3;

  uint32_t ev[KMAX];
  float wt[KMAX];
  bool bad = false;
#pragma unroll
  for (int j = 0; j < KMAX; ++j) {
    wt[j] = 0.f;
    ev[j] = 0u;
    if (j < a.k) {
      const float wj = a.w[t * a.k + j];
      const int32_t e = a.idx[t * a.k + j];
      const bool ok = e >= 0 && e < a.E;
      if (wj != 0.f && !ok) bad = true;
      if (wj != 0.f && ok) {
        wt[j] = wj;
        ev[j] = (uint32_t)e;
      }
    }
  }
  table_dma(a.xt_h, tab4, wv, lane);
  const uint32_t nh = (uint32_t)a.k * C;
  const uint4* hg = (const uint4*)(a.h + (size_t)t * a.k * a.I);
  for (uint32_t c0 = wv * 64; c0 < nh; c0 += MOE_WAVES * 64) {
    const uint32_t c = c0 + lane < nh ? c0 + lane : nh - 1;
    dma16(hg + c, hsh + c0);
  }
  __builtin_amdgcn_sched_barrier(0);

  uint32_t dw[KMAX][R][STEPS][NW];
  uint32_t dbase[KMAX][R];
#pragma unroll
  for (int j = 0; j < KMAX; ++j)
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const uint32_t n = row0 + r;
      const bool rowok = wt[j] != 0.f && n < (uint32_t)a.H;
      dbase[j][r] = rowok ? ev[j] * a.H + n : 0u;
      const uint16_t* drow = a.dc + (size_t)dbase[j][r] * C;
#pragma unroll
      for (int s = 0; s < STEPS; ++s) {
        uint32_t cw = lane * CH + s * 64 * CH;
        cw = cw < C ? cw : 0u;
        load_cw<CH>(drow + cw, dw[j][r][s]);
      }
    }
  __builtin_amdgcn_sched_barrier(0);
  wait_vm<NLOADS>();
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_sched_barrier(0);
  ScaleRaw dsr[KMAX][R][STEPS];
#pragma unroll
  for (int j = 0; j < KMAX; ++j)
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int s = 0; s < STEPS; ++s) {
        uint32_t cw = lane * CH + s * 64 * CH;
        cw = cw < C ? cw : 0u;
        dsr[j][r][s] = scale_raw(a.ds, a.sdt, dbase[j][r] * a.Gi + cw / a.cpg_i);
      }

  float acc[R];
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = 0.f;
#pragma unroll
  for (int j = 0; j < KMAX; ++j) {
    if (wt[j] == 0.f) continue;
#pragma unroll
    for (int s = 0; s < STEPS; ++s) {
      const uint32_t cw0 = lane * CH + s * 64 * CH;
      if (cw0 >= C) continue;
      uint32_t xp[CH][4];
#pragma unroll
      for (int i = 0; i < CH; ++i) {
        permute_x(hsh[j * C + cw0 + i], xp[i]);
      }
#pragma unroll
      for (int r = 0; r < R; ++r) {
        float p = 0.f;
#pragma unroll
        for (int i = 0; i < CH; i += 2) {
          uint32_t ah, al;
          xt_addr<0>(dw[j][r][s][i >> 1], ah, al);
          p = xt_dot<PAIR_BF16>(tab, ah, al, xp[i], p);
          xt_addr<16>(dw[j][r][s][i >> 1], ah, al);
          p = xt_dot<PAIR_BF16>(tab, ah, al, xp[i + 1], p);
        }
        const bool ok = row0 + r < (uint32_t)a.H;
        const uint32_t si = dbase[j][r] * a.Gi + cw0 / a.cpg_i;
        acc[r] = fmaf(ok ? wt[j] * scale_cvt(dsr[j][r][s], a.sdt, si) : 0.f, p, acc[r]);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  }
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const float v = wave_total(acc[r]);
    const uint32_t n = row0 + r;
    if (lane == r && n < (uint32_t)a.H) {
      const float o = bad ? __builtin_nanf("") : v;
      const size_t oi = (size_t)t * a.H + n;
      if (a.odt == KEEP_F16) ((_Float16*)a.out)[oi] = (_Float16)o;
      else if (a.odt == KEEP_BF16) ((uint16_t*)a.out)[oi] = from_float<bf16s>(o).bits;
      else ((float*)a.out)[oi] = o;
    }
  }
}

// ------------------------------------------------------------------ v3: matrix-core layer (one token)
//
// Rows go through v_mfma_f32_16x16x32_{f16,bf16} in tiles of 16. Lane l
// decodes one codeword of tile row l % 16 at codeword slot l / 16 (its H and
// L table entries are exactly the eight operand values of that slot) into
// the B operand; A holds the activation chunk of the same slot, permuted to
// the table's pair order. Gate/up: every A row is the token. Down: A row i is
// route i's SwiGLU output, so one A fragment serves all routes of a block and
// row i of tile i's result is the useful one. Waves split K (256 elements per
// wave) and meet in one small LDS reduction; each wave issues all of its code
// loads before it touches LDS, so the whole code stream of the block is in
// flight while the table is staged.

typedef _Float16 m3h8_t __attribute__((ext_vector_type(8)));
typedef __bf16 m3b8_t __attribute__((ext_vector_type(8)));
typedef float m3f4_t __attribute__((ext_vector_type(4)));

constexpr int M3_MAXW = 16;          // waves per block (K-slices of 256)
constexpr int M3_HCHUNKS = 1544;     // down: k * (I / 8 + 1) h chunks staged in LDS

template <int PK>
__device__ __forceinline__ m3f4_t mfma16(uint4 a, uint4 b, m3f4_t c) {
  if constexpr (PK == PAIR_F16)
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(m3h8_t, a), __builtin_bit_cast(m3h8_t, b), c,
                                                  0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(m3b8_t, a), __builtin_bit_cast(m3b8_t, b), c,
                                                   0, 0, 0);
}

// Codeword in bits [LO, LO + 16) of w -> the B operand: L entry (dims 0,2,4,6)
// then H entry (dims 1,3,5,7), matching permute_x's activation order.
template <int LO>
__device__ __forceinline__ uint4 xt_decode(const char* tab, uint32_t w) {
  uint32_t ah, al;
  xt_addr<LO>(w, ah, al);
  const uint2 eh = *(const uint2*)(tab + ah);
  const uint2 el = *(const uint2*)(tab + al + 0x8000);
  return make_uint4(el.x, el.y, eh.x, eh.y);
}

__device__ __forceinline__ uint32_t dword_of(const uint4& q, int i) {
  return i == 0 ? q.x : i == 1 ? q.y : i == 2 ? q.z : q.w;
}

__device__ __forceinline__ uint4 permuted(const uint4 q) {
  uint32_t xp[4];
  permute_x(q, xp);
  return make_uint4(xp[0], xp[1], xp[2], xp[3]);
}

struct M3Args {
  const void* x;  // [H] fp16 / bf16 (one token)
  int32_t H, I, k, E;
  const int32_t* idx;
  const float* w;
  const uint16_t *gc, *uc, *dc;
  const void *gs, *us, *ds;
  int sdt;
  int32_t Gh, gsz_h, Gi, gsz_i;  // scale groups per row and elements per group
  const uint4* xt;               // expanded table, activation pair kind (gate/up) or bf16 (down)
  float limit;
  uint16_t* h;  // [k, I] bf16, natural order
  void* out;
  int odt;
  int32_t qtiles;  // gate/up: k * I / 16
};

// Block: QT = NT / 2 q-tiles (16 consecutive rows of the flattened [k, I]
// intermediate space), as NT tiles (gate, up, gate, up, ...). H / 256 waves.
template <int PK, int NT>
__global__ __launch_bounds__(1024) void k_moe3_gateup(M3Args a) {
  __shared__ uint4 tab4[XT_BYTES / 16];
  __shared__ uint4 xsh[512];  // the token, natural order (H <= 4096)
  __shared__ float red[M3_MAXW][NT][16];
  constexpr int QT = NT / 2;
  const char* tab = (const char*)tab4;
  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nw = blockDim.x >> 6;
  const uint32_t j = lane & 15, g = lane >> 4;
  const uint32_t C = (uint32_t)a.H >> 3;

  // 0. tiles (scalar)
  uint32_t rbase[QT];
#pragma unroll
  for (int u = 0; u < QT; ++u) {
    const uint32_t qt = blockIdx.x * QT + u;
    const bool valid = qt < (uint32_t)a.qtiles;
    const uint32_t q0 = (valid ? qt : 0u) * 16u;
    const uint32_t route = q0 / (uint32_t)a.I;
    const uint32_t i0 = q0 - route * (uint32_t)a.I;
    const int32_t e = a.idx[route];
    const bool ok = valid && e >= 0 && e < a.E;
    rbase[u] = (ok ? (uint32_t)e * (uint32_t)a.I : 0u) + i0;
  }

  // 1. LDS DMA: table and the token
  for (int i = wv * 64; i < XT_BYTES / 16; i += nw * 64) dma16(a.xt + i + lane, tab4 + i);
  if (wv * 64 < (int)C) dma16((const uint4*)a.x + min(wv * 64 + lane, (int)C - 1), xsh + wv * 64);
  __builtin_amdgcn_sched_barrier(0);

  // 2. codes: 8 codewords (16 B) per lane per tile, exactly NT loads
  const uint32_t kc0 = wv * 32 + g * 8;
  uint4 q[NT];
#pragma unroll
  for (int u = 0; u < QT; ++u) {
    const size_t off = (size_t)(rbase[u] + j) * C + kc0;
    q[2 * u] = *(const uint4*)(a.gc + off);
    q[2 * u + 1] = *(const uint4*)(a.uc + off);
  }
  __builtin_amdgcn_sched_barrier(0);
  wait_vm<NT>();
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_sched_barrier(0);
  // scales of this wave's group (consumed after the decode)
  const uint32_t grp = (uint32_t)(wv * 256) / (uint32_t)a.gsz_h;
  ScaleRaw sr[NT];
#pragma unroll
  for (int u = 0; u < QT; ++u) {
    const uint32_t si = (rbase[u] + j) * (uint32_t)a.Gh + grp;
    sr[2 * u] = scale_raw(a.gs, a.sdt, si);
    sr[2 * u + 1] = scale_raw(a.us, a.sdt, si);
  }

  // 3. decode into B, token chunk in A
  m3f4_t acc[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) acc[t] = m3f4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int m = 0; m < 8; ++m) {
    const uint4 A = permuted(xsh[kc0 + m]);
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const uint32_t wd = dword_of(q[t], m >> 1);
      const uint4 B = (m & 1) ? xt_decode<16>(tab, wd) : xt_decode<0>(tab, wd);
      acc[t] = mfma16<PK>(A, B, acc[t]);
    }
  }

  // 4. scaled per-wave partials (every A row holds the token: D row 0 is the dot)
#pragma unroll
  for (int u = 0; u < QT; ++u) {
    const uint32_t si = (rbase[u] + j) * (uint32_t)a.Gh + grp;
    if (lane < 16) {
      red[wv][2 * u][j] = acc[2 * u][0] * scale_cvt(sr[2 * u], a.sdt, si);
      red[wv][2 * u + 1][j] = acc[2 * u + 1][0] * scale_cvt(sr[2 * u + 1], a.sdt, si);
    }
  }
  __syncthreads();

  // 5. wave sum, SwiGLU, h (bf16, natural order)
  if (threadIdx.x < QT * 16) {
    const uint32_t u = threadIdx.x >> 4, jj = threadIdx.x & 15;
    const uint32_t qt = blockIdx.x * QT + u;
    float gsum = 0.f, usum = 0.f;
    for (int w = 0; w < nw; ++w) {
      gsum += red[w][2 * u][jj];
      usum += red[w][2 * u + 1][jj];
    }
    if (qt < (uint32_t)a.qtiles) {
      const uint32_t q0 = qt * 16u;
      const uint32_t route = q0 / (uint32_t)a.I;
      const int32_t e = a.idx[route];
      if (e >= 0 && e < a.E) a.h[q0 + jj] = from_float<bf16s>(silu_mul(gsum, usum, a.limit)).bits;
    }
  }
}

// Block: 16 output rows (blockIdx.x * 16 ..) over every route; I / 256 waves.
// 16-byte load through the global address space (a pointer chosen at run time
// would otherwise be a flat access, which the compiler must also count as
// LDS traffic and so waits for far too conservatively).
__device__ __forceinline__ uint4 ldg16(const void* p) {
  typedef unsigned int v4u __attribute__((ext_vector_type(4)));
  const v4u v = *(const __attribute__((address_space(1))) v4u*)p;
  return uint4{v.x, v.y, v.z, v.w};
}

// Block barrier for LDS traffic only: unlike __syncthreads it does not wait
// for this wave's outstanding global loads (the code stream keeps flowing).
__device__ __forceinline__ void lds_barrier() { rt_lds_barrier(); }

// Every block copies the same 128 KiB table (128 pieces of 1 KiB) into its
// LDS. Blocks are dealt round-robin to the 8 XCDs, so blocks b, b + 8, ...
// share one L2: each starts at its own piece, so that at any moment they
// request different lines and most requests hit a line another block of the
// XCD already brought in, instead of all missing on the same line together.
__device__ __forceinline__ uint32_t xt_rotation() { return ((blockIdx.x >> 3) * 4u) & 127u; }

template <int KMAX>
__global__ __launch_bounds__(512) void k_moe3_down(M3Args a) {
  __shared__ uint4 tab4[XT_BYTES / 16];
  __shared__ uint4 hsh[M3_HCHUNKS];  // route r's h at r * (I / 8 + 1): the pad spreads routes over banks
  __shared__ float red[8][KMAX][16];
  const char* tab = (const char*)tab4;
  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // 8 waves; I / 256 of them decode
  const int nwd = a.I >> 8;
  const uint32_t j = lane & 15, g = lane >> 4;
  const uint32_t C = (uint32_t)a.I >> 3, S = C + 1;
  const uint32_t n0 = blockIdx.x * 16;

  // 1. the routes (scalar loads: KMAX == k, so all in bounds), then the bf16
  //    table, which does not depend on them (16 DMA ops per wave)
  int32_t e_r[KMAX];
  float w_r[KMAX];
#pragma unroll
  for (int r = 0; r < KMAX; ++r) {
    e_r[r] = a.idx[r];
    w_r[r] = a.w[r];
  }
  const uint32_t rot = xt_rotation();
#pragma unroll
  for (int i = 0; i < XT_BYTES / 16 / 512; ++i) {
    const uint32_t piece = ((uint32_t)(i * 8 + wv) + rot) & 127u;
    dma16(a.xt + piece * 64 + lane, tab4 + piece * 64);
  }
  __builtin_amdgcn_sched_barrier(0);
  uint32_t dbase[KMAX];
  float wt[KMAX];
  bool bad = false;
#pragma unroll
  for (int r = 0; r < KMAX; ++r) {
    const bool ok = e_r[r] >= 0 && e_r[r] < a.E;
    bad |= w_r[r] != 0.f && !ok;
    wt[r] = ok ? w_r[r] : 0.f;
    dbase[r] = (ok ? (uint32_t)e_r[r] * (uint32_t)a.H : 0u) + n0;
  }

  // 3. every route's h (pieces of 64 chunks, (KMAX + 1) / 2 DMA ops per wave;
  //    unused slots repeat a valid piece), then the scales and the codes
  {
    const uint32_t per_route = C / 64u, npieces = (uint32_t)KMAX * per_route;
#pragma unroll
    for (int i = 0; i < (KMAX + 1) / 2; ++i) {
      uint32_t p = (uint32_t)wv + 8u * i;
      p = p < npieces ? p : p % npieces;
      const uint32_t r = p / per_route, c0 = (p - r * per_route) * 64u;
      dma16((const uint4*)(a.h + (size_t)r * a.I) + c0 + lane, hsh + r * S + c0);
    }
  }
  const bool dec = wv < nwd;  // wave-uniform
  const uint32_t kc0 = (dec ? wv : 0) * 32 + g * 8;
  const uint32_t grp = (uint32_t)((dec ? wv : 0) * 256) / (uint32_t)a.gsz_i;
  ScaleRaw sr[KMAX];
#pragma unroll
  for (int r = 0; r < KMAX; ++r) sr[r] = scale_raw(a.ds, a.sdt, (dbase[r] + j) * (uint32_t)a.Gi + grp);
  // route r's codes are loaded PD routes ahead of its decode (see the gate/up kernel)
  constexpr int PD = 3;
  uint4 q[KMAX];
  auto load_route = [&](int r) { q[r] = ldg16(a.dc + (size_t)(dbase[r] + j) * C + kc0); };
#pragma unroll
  for (int r = 0; r < PD && r < KMAX; ++r) load_route(r);  // every wave: the wait below counts them
  __builtin_amdgcn_sched_barrier(0);
  wait_vm<KMAX + (PD < KMAX ? PD : KMAX)>();  // the table and h DMAs, not the scales and codes behind them
  lds_barrier();

  // 4. decode, route by route; A row i holds route i's h
  if (dec) {
    const uint32_t ri = j < (uint32_t)KMAX ? j : 0u;
    uint4 A[8];
#pragma unroll
    for (int m = 0; m < 8; ++m) A[m] = permuted(hsh[ri * S + kc0 + m]);
#pragma unroll
    for (int r = 0; r < KMAX; ++r) {  // branch-free: zero-weight routes are dropped in the sum
      if (r + PD < KMAX) load_route(r + PD);
      __builtin_amdgcn_sched_barrier(0);
      m3f4_t acc = m3f4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int m = 0; m < 8; ++m) {
        const uint32_t wd = dword_of(q[r], m >> 1);
        const uint4 B = (m & 1) ? xt_decode<16>(tab, wd) : xt_decode<0>(tab, wd);
        acc = mfma16<PAIR_BF16>(A[m], B, acc);
      }
      // route r's dot is D row r: lanes 16 * (r / 4) + j, register r % 4
      if (g == (uint32_t)(r >> 2))
        red[wv][r][j] = acc[r & 3] * scale_cvt(sr[r], a.sdt, (dbase[r] + j) * (uint32_t)a.Gi + grp);
    }
  }
  lds_barrier();

  // 5. weighted sum over routes and waves
  if (threadIdx.x < 16) {
    float o = 0.f;
#pragma unroll
    for (int r = 0; r < KMAX; ++r) {
      float v = 0.f;
      for (int w = 0; w < nwd; ++w) v += red[w][r][threadIdx.x];
      o = wt[r] != 0.f ? fmaf(wt[r], v, o) : o;
    }
    if (bad) o = __builtin_nanf("");
    const size_t oi = n0 + threadIdx.x;
    if (a.odt == KEEP_F16) ((_Float16*)a.out)[oi] = (_Float16)o;
    else if (a.odt == KEEP_BF16) ((uint16_t*)a.out)[oi] = from_float<bf16s>(o).bits;
    else ((float*)a.out)[oi] = o;
  }
  wait_vm<0>();  // no DMA into this block's LDS may outlive it
}

// ------------------------------------------------------------------ host

struct GuShape {
  int waves, r;
};

// (waves per block, rows per wave): waves * R must divide the per-token row
// count (a block never straddles a token); prefer exactly filling 256 CUs.
static GuShape pick_gu(int64_t rows_per_token, int64_t total_rows) {
  const GuShape cands[] = {{16, 3}, {8, 6}, {16, 2}, {8, 4}, {16, 1}, {8, 3}, {8, 2}, {8, 1}};
  GuShape best{0, 0};
  double best_eff = -1.0;
  for (const GuShape c : cands) {
    if (rows_per_token % (c.waves * c.r)) continue;
    const int64_t units = total_rows / c.r;
    const int64_t blocks = (units + c.waves - 1) / c.waves;
    const int64_t rounds = (blocks + 255) / 256;
    const double eff = (double)units / (double)(rounds * 256 * c.waves);
    if (eff > best_eff + 1e-9) {
      best_eff = eff;
      best = c;
    }
  }
  return best;
}

bool moe_v2_supported(int64_t H, int64_t I, int64_t k, int64_t group_h, int64_t group_i) {
  const int64_t Ch = H / 8, Ci = I / 8;
  const bool gu = Ch == 1024 || Ch == 512 || Ch == 256 || Ch == 128;
  const bool dn = Ci == 512 || Ci == 256 || Ci == 192 || Ci == 128;
  const bool groups = (group_h / 8) % 8 == 0 && (group_i / 8) % 8 == 0;
  return gu && dn && groups && k >= 1 && k <= 8 && k * Ci <= 1536 && pick_gu(k * I, k * I).r > 0;
}

template <int PK, int NWAV, int R>
static void launch_gateup_r(const MoeV2Args& a, hipStream_t s) {
  const int64_t C = a.H / 8;
  const dim3 grid((unsigned)((a.units + NWAV - 1) / NWAV)), blk(NWAV * 64);
  if (C == 1024) hipLaunchKernelGGL((k_moe_gateup_v2<PK, NWAV, R, 8, 2>), grid, blk, 0, s, a);
  else if (C == 512) hipLaunchKernelGGL((k_moe_gateup_v2<PK, NWAV, R, 8, 1>), grid, blk, 0, s, a);
  else if (C == 256) hipLaunchKernelGGL((k_moe_gateup_v2<PK, NWAV, R, 4, 1>), grid, blk, 0, s, a);
  else hipLaunchKernelGGL((k_moe_gateup_v2<PK, NWAV, R, 2, 1>), grid, blk, 0, s, a);
}

template <int PK>
static void launch_gateup_v2(const MoeV2Args& a, GuShape g, hipStream_t s) {
  if (g.waves == 16) {
    if (g.r == 3) launch_gateup_r<PK, 16, 3>(a, s);
    else if (g.r == 2) launch_gateup_r<PK, 16, 2>(a, s);
    else launch_gateup_r<PK, 16, 1>(a, s);
  } else {
    if (g.r == 6) launch_gateup_r<PK, 8, 6>(a, s);
    else if (g.r == 4) launch_gateup_r<PK, 8, 4>(a, s);
    else if (g.r == 3) launch_gateup_r<PK, 8, 3>(a, s);
    else if (g.r == 2) launch_gateup_r<PK, 8, 2>(a, s);
    else launch_gateup_r<PK, 8, 1>(a, s);
  }
}

static void launch_down_v2(const MoeV2Args& a, int R, hipStream_t s) {
  const int64_t C = a.I / 8;
  const int64_t bpt = (a.H + MOE_WAVES * R - 1) / (MOE_WAVES * R);
  const dim3 grid((unsigned)(bpt * a.T)), blk(MOE_THREADS);
#define DN(RR, CHH, ST) hipLaunchKernelGGL((k_moe_down_v2<RR, CHH, ST, 8>), grid, blk, 0, s, a)
  if (R == 1) {
    if (C == 512) DN(1, 8, 1);
    else if (C == 256 || C == 192) DN(1, 4, 1);
    else DN(1, 2, 1);
  } else {
    if (C == 512) DN(2, 8, 1);
    else if (C == 256 || C == 192) DN(2, 4, 1);
    else DN(2, 2, 1);
  }
#undef DN
}

int moe_v2_launch(bool gateup, bool down, const void* x, int x_dtype, int64_t T, int64_t H, int64_t I,
                  const int32_t* idx, const float* w, int64_t k, int64_t E, const uint16_t* gc, const void* gs,
                  const uint16_t* uc, const void* us, const uint16_t* dc, const void* ds, int sdt, int64_t group_h,
                  int64_t group_i, const void* prepared, float limit, void* h, void* out, int odt, hipStream_t s) {
  MoeV2Args a{};
  a.x = x; a.T = (int32_t)T; a.H = (int32_t)H; a.I = (int32_t)I; a.k = (int32_t)k; a.E = (int32_t)E;
  a.idx = idx; a.w = w; a.gc = gc; a.uc = uc; a.dc = dc; a.gs = gs; a.us = us; a.ds = ds; a.sdt = sdt;
  a.Gh = (int32_t)(H / group_h); a.cpg_h = (int32_t)(group_h / 8); a.Gi = (int32_t)(I / group_i);
  a.cpg_i = (int32_t)(group_i / 8);
  a.xt_x = (const uint4*)((const char*)prepared + (x_dtype == KEEP_BF16 ? XT_BYTES : 0));
  a.xt_h = (const uint4*)((const char*)prepared + XT_BYTES);
  a.limit = limit; a.h = (uint16_t*)h; a.out = out; a.odt = odt;
  a.rows_per_token = (int32_t)(k * I);
  if (gateup) {
    const GuShape g = pick_gu(k * I, T * k * I);
    a.units = (int32_t)(T * k * I / g.r);
    if (x_dtype == KEEP_BF16) launch_gateup_v2<PAIR_BF16>(a, g, s);
    else launch_gateup_v2<PAIR_F16>(a, g, s);
  }
  if (down) {
    const int Rd = (H / MOE_WAVES) * T >= 256 * 2 ? 2 : 1;
    launch_down_v2(a, Rd, s);
  }
  return 0;
}


// ------------------------------------------------------------------ v3 host

static int m3_qt(int64_t qtiles) {
  const int64_t qt = (qtiles + 255) / 256;
  return (int)(qt < 1 ? 1 : qt);
}

bool moe_v3_gateup_supported(int64_t T, int64_t H, int64_t I, int64_t k, int64_t group_h) {
  return T == 1 && H % 256 == 0 && H >= 256 && H <= 4096 && I % 16 == 0 && k >= 1 && group_h % 256 == 0 &&
         m3_qt(k * I / 16) <= 4;
}

bool moe_v3_down_supported(int64_t T, int64_t H, int64_t I, int64_t k, int64_t group_i) {
  return T == 1 && H % 16 == 0 && I % 512 == 0 && I <= 2048 && k >= 1 && k <= 8 && k * (I / 8 + 1) <= M3_HCHUNKS &&
         group_i % 256 == 0;
}

void moe_v3_launch(bool gateup, bool down, const void* x, int x_dtype, int64_t H, int64_t I, const int32_t* idx,
                   const float* w, int64_t k, int64_t E, const uint16_t* gc, const void* gs, const uint16_t* uc,
                   const void* us, const uint16_t* dc, const void* ds, int sdt, int64_t group_h, int64_t group_i,
                   const void* prepared, float limit, void* h, void* out, int odt, hipStream_t s) {
  M3Args a{};
  a.x = x; a.H = (int32_t)H; a.I = (int32_t)I; a.k = (int32_t)k; a.E = (int32_t)E; a.idx = idx; a.w = w;
  a.gc = gc; a.uc = uc; a.dc = dc; a.gs = gs; a.us = us; a.ds = ds; a.sdt = sdt;
  a.Gh = (int32_t)(H / group_h); a.gsz_h = (int32_t)group_h; a.Gi = (int32_t)(I / group_i);
  a.gsz_i = (int32_t)group_i; a.limit = limit; a.h = (uint16_t*)h; a.out = out; a.odt = odt;
  a.qtiles = (int32_t)(k * I / 16);
  if (gateup) {
    a.xt = (const uint4*)((const char*)prepared + (x_dtype == KEEP_BF16 ? XT_BYTES : 0));
    const int qt = m3_qt(a.qtiles);
    const dim3 grid((unsigned)((a.qtiles + qt - 1) / qt)), blk((unsigned)(H / 256 * 64));
#define GU(PK, NT) hipLaunchKernelGGL((k_moe3_gateup<PK, NT>), grid, blk, 0, s, a)
    if (x_dtype == KEEP_BF16) {
      if (qt == 1) GU(PAIR_BF16, 2); else if (qt == 2) GU(PAIR_BF16, 4); else if (qt == 3) GU(PAIR_BF16, 6);
      else GU(PAIR_BF16, 8);
    } else {
      if (qt == 1) GU(PAIR_F16, 2); else if (qt == 2) GU(PAIR_F16, 4); else if (qt == 3) GU(PAIR_F16, 6);
      else GU(PAIR_F16, 8);
    }
#undef GU
  }
  if (down) {
    a.xt = (const uint4*)((const char*)prepared + XT_BYTES);
    const dim3 grid((unsigned)(H / 16)), blk(512u);
    switch (k) {
      case 1: hipLaunchKernelGGL((k_moe3_down<1>), grid, blk, 0, s, a); break;
      case 2: hipLaunchKernelGGL((k_moe3_down<2>), grid, blk, 0, s, a); break;
      case 3: hipLaunchKernelGGL((k_moe3_down<3>), grid, blk, 0, s, a); break;
      case 4: hipLaunchKernelGGL((k_moe3_down<4>), grid, blk, 0, s, a); break;
      case 5: hipLaunchKernelGGL((k_moe3_down<5>), grid, blk, 0, s, a); break;
      case 6: hipLaunchKernelGGL((k_moe3_down<6>), grid, blk, 0, s, a); break;
      case 7: hipLaunchKernelGGL((k_moe3_down<7>), grid, blk, 0, s, a); break;
      default: hipLaunchKernelGGL((k_moe3_down<8>), grid, blk, 0, s, a); break;
    }
  }
}


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
constexpr int PREPARED_TOTAL = 2 * XT_BYTES + 4096 + 256 + 65536;  // expanded tables, int8 tables, flag, LDS image

}  // namespace keep

using namespace keep;

extern "C" int keep_e8p_prepare(const uint32_t* table, void* prepared, void* stream) {
  KEEP_REQUIRE(table && prepared, "table and prepared must be non-null");
  KEEP_REQUIRE(aligned(prepared, 16), "prepared must be 16-byte aligned");
  hipStream_t s = (hipStream_t)stream;
  hipLaunchKernelGGL((k_expand_table<PAIR_F16>), dim3(XT_ENTRIES / 256), dim3(256), 0, s, table, (uint2*)prepared);
  hipLaunchKernelGGL((k_expand_table<PAIR_BF16>), dim3(XT_ENTRIES / 256), dim3(256), 0, s, table,
                     (uint2*)((char*)prepared + XT_BYTES));
  tq_build(table, prepared, s);
  return launch_status("keep_e8p_prepare");
}

extern "C" int keep_e8p_prepared_bytes(void) { return PREPARED_TOTAL; }

extern "C" int keep_moe_layer_supported(int64_t E, int64_t H, int64_t I, int64_t k, int64_t group_size_h,
                                        int64_t group_size_i) {
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
