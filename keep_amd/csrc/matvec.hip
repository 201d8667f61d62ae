// Routed E8P mat-vec family for gfx950: decode (M = 1), verify rows (few
// tokens) and the fused SwiGLU MoE decode layer.
//
// Layout: one wave64 owns MV_ROWS output rows of one route. Lanes split the
// K axis in chunks of CH codewords (CH*2 bytes: 16 B loads when CH = 8), so a
// wave reads MV_ROWS contiguous 64*CH*2-byte spans per step, fully coalesced.
// The lane's activation chunk is loaded once and reused for all MV_ROWS rows.
// Each block (4 waves) first builds the 256-entry codebook as packed fp16 or
// bf16 pairs in LDS (4 KiB). Accumulation is fp32: per chunk a partial dot,
// times the row's group scale, added to the row accumulator; then a fixed
// butterfly over the 64 lanes. Every kernel in this file that shares this
// order (mat-vec, verify tiles) is bit-identical per route.
#include "common.h"

namespace keep {

constexpr int MV_WAVES = 4;
constexpr int MV_ROWS = 2;
constexpr uint32_t NO_RESIDUAL = 0xffffffffu;

__device__ __forceinline__ float scale_at(const void* p, int dt, int64_t i) {
  if (dt == KEEP_F16) return (float)((const _Float16*)p)[i];
  if (dt == KEEP_BF16) return __uint_as_float((uint32_t)((const uint16_t*)p)[i] << 16);
  return ((const float*)p)[i];
}

// The raw bits of scale i (loaded in one place whatever the dtype, so the
// load can stay in flight) and their value; scale_of_bits(scale_bits(..))
// equals scale_at(..).
__device__ __forceinline__ uint32_t scale_bits(const void* p, int dt, int64_t i) {
  if (dt == KEEP_F32) return ((const uint32_t*)p)[i];
  return ((const uint16_t*)p)[i];
}
__device__ __forceinline__ float scale_of_bits(uint32_t b, int dt) {
  if (dt == KEEP_F16) return (float)__builtin_bit_cast(_Float16, (uint16_t)b);
  if (dt == KEEP_BF16) return __uint_as_float(b << 16);
  return __uint_as_float(b);
}

__device__ __forceinline__ void store_at(void* p, int dt, int64_t i, float v) {
  if (dt == KEEP_F16) ((_Float16*)p)[i] = (_Float16)v;
  else if (dt == KEEP_BF16) ((uint16_t*)p)[i] = from_float<bf16s>(v).bits;
  else ((float*)p)[i] = v;
}

template <int R>
__device__ __forceinline__ float select_row(const float (&v)[R], int i) {
  float out = v[0];
#pragma unroll
  for (int r = 1; r < R; ++r) out = (i == r) ? v[r] : out;
  return out;
}

// ------------------------------------------------------------------ E8P decode

template <int PK>
__global__ __launch_bounds__(256) void k_e8p_decode(const uint16_t* codes, int64_t n, const uint32_t* table,
                                                    const void* scales, int sdt, int64_t cpr, int64_t gcw,
                                                    float* out) {
  __shared__ uint4 tab[256];
  build_codebook<16, PK>(tab, table);
  __syncthreads();
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    const uint32_t c = codes[i];
    const E8PSigns sg = e8p_signs(c);
    const uint4 e = tab[c >> 8];
    const uint32_t w[4] = {e.x ^ sg.m0, e.y ^ sg.m1, e.z ^ sg.m2, e.w ^ sg.m3};
    float s = 1.f;
    if (scales) {
      const int64_t row = i / cpr, cw = i - row * cpr;
      s = scale_at(scales, sdt, row * (cpr / gcw) + cw / gcw);
    }
    float v[8];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      v[2 * k] = (pair_lo<PK>(w[k]) + sg.shift) * s;
      v[2 * k + 1] = (pair_hi<PK>(w[k]) + sg.shift) * s;
    }
    float4* o = (float4*)(out + i * 8);
    o[0] = make_float4(v[0], v[1], v[2], v[3]);
    o[1] = make_float4(v[4], v[5], v[6], v[7]);
  }
}

// 8-bit E8 decode: code byte c -> the packed entry table[c], nibble d = dim d,
// value (nibble - 8) / 2 (exact in fp32), times the group scale.
__global__ __launch_bounds__(256) void k_e8_decode(const uint8_t* codes, int64_t n, const uint32_t* table,
                                                   const void* scales, int sdt, int64_t cpr, int64_t gcw,
                                                   float* out) {
  __shared__ uint32_t tab[256];
  tab[threadIdx.x] = table[threadIdx.x];
  __syncthreads();
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    const uint32_t p = tab[codes[i]];
    float s = 1.f;
    if (scales) {
      const int64_t row = i / cpr, cw = i - row * cpr;
      s = scale_at(scales, sdt, row * (cpr / gcw) + cw / gcw);
    }
    float v[8];
#pragma unroll
    for (int d = 0; d < 8; ++d) v[d] = ((float)((p >> (4 * d)) & 15u) - 8.f) * 0.5f * s;
    float4* o = (float4*)(out + i * 8);
    o[0] = make_float4(v[0], v[1], v[2], v[3]);
    o[1] = make_float4(v[4], v[5], v[6], v[7]);
  }
}

// ------------------------------------------------------------------ routed mat-vec

struct MatvecArgs {
  const void* x;
  int64_t x_rows;
  const void* codes;
  const void* scales;
  int sdt;
  const uint32_t* table;
  const int32_t* rhs;
  const int32_t* lhs;
  int64_t routes, x_div;
  int64_t E, N, K, G, cpg;
  const uint8_t* rcodes;
  const void* rscales;
  int64_t rG, rcpg;
  const uint32_t* rtable;
  const uint32_t* hot;
  int64_t nhot;
  void* out;
  int odt;
  int64_t row_blocks;
  int zero_none;  // a route whose index is 0xFFFFFFFF writes zeros (the residual-only form)
};

template <int CB, typename XT, int CH, bool NESTED>
__global__ __launch_bounds__(256) void k_vq_matvec(MatvecArgs a) {
  constexpr int PK = PairOf<XT>::value;
  constexpr int NW = (CH * CB / 8 + 3) / 4;
  constexpr int RNW = (CH + 3) / 4;
  __shared__ uint4 tab[256];
  __shared__ uint4 rtab[NESTED ? 256 : 1];
  const int lane = threadIdx.x & 63;
  const int wv = threadIdx.x >> 6;
  const int64_t route = blockIdx.x / a.row_blocks;
  const int64_t rb = blockIdx.x - route * a.row_blocks;
  const int64_t row0 = (rb * MV_WAVES + wv) * MV_ROWS;
  const bool live = row0 < a.N;
  // The route's expert and activation row, then the first chunk's codes,
  // scales and activations are in flight while the codebook is built.
  const int64_t e = a.rhs ? (int64_t)a.rhs[route] : 0;  // no route vector: one matrix, no dependent load
  const int64_t xr = a.lhs ? (int64_t)a.lhs[route] : route / a.x_div;
  uint32_t hot = NO_RESIDUAL;
  bool bad = e < 0 || e >= a.E || xr < 0 || xr >= a.x_rows;
  if constexpr (NESTED) {
    if (!bad) {
      hot = a.hot[e];
      bad = hot != NO_RESIDUAL && (int64_t)hot >= a.nhot;
    }
  }
  const int64_t C = a.K >> 3;
  const XT* xrow = (const XT*)a.x + xr * a.K;
  const char* cbase = (const char*)a.codes + (e * a.N) * C * (CB / 8);
  uint32_t words[MV_ROWS][NW], sb[MV_ROWS];
  XChunk<XT, CH> xc;
  auto load_chunk = [&](int64_t cw) {  // rows past N load row N - 1 and are never used
    const int64_t g = cw / a.cpg;
#pragma unroll
    for (int r = 0; r < MV_ROWS; ++r) {
      const int64_t row = row0 + r < a.N ? row0 + r : a.N - 1;
      load_codes<CB, CH>(cbase + row * C * (CB / 8), cw, words[r]);
      sb[r] = scale_bits(a.scales, a.sdt, (e * a.N + row) * a.G + g);
    }
    xc.load(xrow, cw);
  };
  const uint32_t tpk = a.table[threadIdx.x];  // blockDim.x == 256: one codebook entry per thread
  int64_t cw = (int64_t)lane * CH;
  if (live && !bad && cw < C) load_chunk(cw);
  codebook_entry<CB, PK>(tab, threadIdx.x, tpk);
  if constexpr (NESTED) load_pair_table<PK>(rtab, a.rtable);
  __syncthreads();
  if (!live) return;
  if (bad) {
    const float fill = a.zero_none && e == -1 ? 0.f : __builtin_nanf("");
    if (lane < MV_ROWS && row0 + lane < a.N) store_at(a.out, a.odt, route * a.N + row0 + lane, fill);
    return;
  }
  float acc[MV_ROWS], racc[MV_ROWS];
#pragma unroll
  for (int r = 0; r < MV_ROWS; ++r) acc[r] = racc[r] = 0.f;

  for (; cw < C; cw += 64 * CH) {
#pragma unroll
    for (int r = 0; r < MV_ROWS; ++r) {
      if (row0 + r < a.N) {
        const float part = chunk_dot<CB, XT, CH>(words[r], tab, xc);
        acc[r] += part * scale_of_bits(sb[r], a.sdt);
      }
    }
    if constexpr (NESTED) {
      if (hot != NO_RESIDUAL) {
        const int64_t rg = cw / a.rcpg;
        const char* rbase = (const char*)a.rcodes + ((int64_t)hot * a.N) * C;
#pragma unroll
        for (int r = 0; r < MV_ROWS; ++r) {
          const int64_t row = row0 + r;
          if (row < a.N) {
            uint32_t rw[RNW];
            load_codes<8, CH>(rbase + row * C, cw, rw);
            const float part = chunk_dot<8, XT, CH>(rw, rtab, xc);
            racc[r] += part * scale_at(a.rscales, a.sdt, ((int64_t)hot * a.N + row) * a.rG + rg);
          }
        }
      }
    }
    if (cw + 64 * CH < C) load_chunk(cw + 64 * CH);
  }
#pragma unroll
  for (int r = 0; r < MV_ROWS; ++r) {
    acc[r] = wave_sum(acc[r]);
    if constexpr (NESTED) {
      if (hot != NO_RESIDUAL) acc[r] += wave_sum(racc[r]);
    }
  }
  if (lane < MV_ROWS && row0 + lane < a.N) store_at(a.out, a.odt, route * a.N + row0 + lane, select_row(acc, lane));
}

// ------------------------------------------------------------------ expert-grouped verify tiles

struct TileArgs {
  const void* x;
  int64_t x_rows;
  const void* codes;
  const void* scales;
  int sdt;
  const uint32_t* table;
  const int32_t* lhs;
  int64_t routes;
  const int32_t *te, *to, *tc;
  int64_t n_tiles, m_rows;
  int64_t E, N, K, G, cpg;
  void* out;
  int odt;
  int64_t row_blocks;
};

// One wave: MV_ROWS rows of one expert for up to m_rows routes. Codes
// (CB = 16: E8P uint16, CB = 8: 8-bit E8 uint8) are loaded and kept in
// registers once; each route re-reads only its own activation chunk (L1/L2
// resident). Per route, the lane order and the chunk/scale/butterfly
// sequence equal k_vq_matvec's, so results are bit-identical with the flat
// mat-vec.
template <int CB, typename XT, int CH>
__global__ __launch_bounds__(256) void k_vq_matvec_tiles(TileArgs a) {
  constexpr int PK = PairOf<XT>::value;
  constexpr int NW = (CH * CB / 8 + 3) / 4;
  constexpr int MMAX = 8;
  __shared__ uint4 tab[256];
  const int lane = threadIdx.x & 63;
  const int wv = threadIdx.x >> 6;
  const int64_t tile = blockIdx.x / a.row_blocks;
  const int64_t rb = blockIdx.x - tile * a.row_blocks;
  const int64_t row0 = (rb * MV_WAVES + wv) * MV_ROWS;
  // The tile, then its first chunk's codes and scales are in flight while
  // the codebook is built.
  const int cnt = a.tc[tile];
  const int64_t off = a.to[tile];
  const int64_t e = a.te[tile];
  const int m = cnt < (int)a.m_rows ? cnt : (int)a.m_rows;
  const bool live = row0 < a.N && cnt > 0;
  const bool bad = e < 0 || e >= a.E || off < 0 || off + m > a.routes;
  const int64_t C = a.K >> 3;
  const char* cbase = (const char*)a.codes + (e * a.N) * C * (CB / 8);
  uint32_t words[MV_ROWS][NW], sb[MV_ROWS];
  auto load_chunk = [&](int64_t cw) {  // rows past N load row N - 1 and are never used
    const int64_t g = cw / a.cpg;
#pragma unroll
    for (int r = 0; r < MV_ROWS; ++r) {
      const int64_t row = row0 + r < a.N ? row0 + r : a.N - 1;
      load_codes<CB, CH>(cbase + row * C * (CB / 8), cw, words[r]);
      sb[r] = scale_bits(a.scales, a.sdt, (e * a.N + row) * a.G + g);
    }
  };
  const uint32_t tpk = a.table[threadIdx.x];  // blockDim.x == 256: one codebook entry per thread
  int64_t cw = (int64_t)lane * CH;
  if (live && !bad && cw < C) load_chunk(cw);
  codebook_entry<CB, PK>(tab, threadIdx.x, tpk);
  __syncthreads();
  if (!live) return;
  if (bad) {
    for (int i = 0; i < m && off + i < a.routes && off + i >= 0; ++i)
      if (lane < MV_ROWS && row0 + lane < a.N) store_at(a.out, a.odt, (off + i) * a.N + row0 + lane, __builtin_nanf(""));
    return;
  }
  int64_t xr[MMAX];
#pragma unroll
  for (int i = 0; i < MMAX; ++i) {
    int64_t v = i < m ? (int64_t)a.lhs[off + i] : 0;
    xr[i] = (v < 0 || v >= a.x_rows) ? -1 : v;
  }
  float acc[MMAX][MV_ROWS];
#pragma unroll
  for (int i = 0; i < MMAX; ++i)
#pragma unroll
    for (int r = 0; r < MV_ROWS; ++r) acc[i][r] = 0.f;

  for (; cw < C; cw += 64 * CH) {
#pragma unroll
    for (int i = 0; i < MMAX; ++i) {
      if (i < m && xr[i] >= 0) {
        XChunk<XT, CH> xc;
        xc.load((const XT*)a.x + xr[i] * a.K, cw);
#pragma unroll
        for (int r = 0; r < MV_ROWS; ++r) {
          if (row0 + r < a.N) acc[i][r] += chunk_dot<CB, XT, CH>(words[r], tab, xc) * scale_of_bits(sb[r], a.sdt);
        }
      }
    }
    if (cw + 64 * CH < C) load_chunk(cw + 64 * CH);
  }
#pragma unroll
  for (int i = 0; i < MMAX; ++i) {
    if (i < m) {
#pragma unroll
      for (int r = 0; r < MV_ROWS; ++r) acc[i][r] = wave_sum(acc[i][r]);
      const float v = xr[i] >= 0 ? select_row(acc[i], lane) : __builtin_nanf("");
      if (lane < MV_ROWS && row0 + lane < a.N) store_at(a.out, a.odt, (off + i) * a.N + row0 + lane, v);
    }
  }
}

// ------------------------------------------------------------------ fused MoE decode

struct MoeArgs {
  const void* x;
  int64_t T, H, I;
  const int32_t* idx;
  const float* w;
  int64_t k, E;
  const uint16_t *gc, *uc, *dc;
  const void *gs, *us, *ds;
  int sdt;
  int64_t Gh, cpg_h, Gi, cpg_i;
  const uint32_t* table;
  float limit;
  void* h;
  void* out;
  int odt;
  int64_t rb_gu, rb_d;
};

__device__ __forceinline__ float swiglu(float g, float u, float limit) {
  if (limit > 0.f) {
    g = fminf(g, limit);
    u = fminf(fmaxf(u, -limit), limit);
  }
  return g / (1.f + __expf(-g)) * u;
}

// Gate and up for MV_ROWS intermediate rows of one route, then SwiGLU in
// fp32; h is stored as bf16 (the SwiGLU product of unit-scale activations can
// exceed the fp16 range; bf16 keeps fp32's exponent, as the reference's
// serving step does). A route with weight 0 is skipped (its h is never read).
template <typename XT, int CH>
__global__ __launch_bounds__(256) void k_moe_gateup(MoeArgs a) {
  constexpr int PK = PairOf<XT>::value;
  constexpr int NW = (CH * 2 + 3) / 4;
  __shared__ uint4 tab[256];
  build_codebook<16, PK>(tab, a.table);
  __syncthreads();
  const int lane = threadIdx.x & 63;
  const int wv = threadIdx.x >> 6;
  const int64_t route = blockIdx.x / a.rb_gu;
  const int64_t rb = blockIdx.x - route * a.rb_gu;
  const int64_t row0 = (rb * MV_WAVES + wv) * MV_ROWS;
  if (row0 >= a.I) return;
  if (a.w[route] == 0.f) return;
  const int64_t t = route / a.k;
  const int64_t e = a.idx[route];
  bf16s* hrow = (bf16s*)a.h + route * a.I;
  if (e < 0 || e >= a.E) {
    if (lane < MV_ROWS && row0 + lane < a.I) hrow[row0 + lane] = from_float<bf16s>(__builtin_nanf(""));
    return;
  }
  const int64_t C = a.H >> 3;
  const XT* xrow = (const XT*)a.x + t * a.H;
  const char* gbase = (const char*)a.gc + (e * a.I) * C * 2;
  const char* ubase = (const char*)a.uc + (e * a.I) * C * 2;
  float ag[MV_ROWS], au[MV_ROWS];
#pragma unroll
  for (int r = 0; r < MV_ROWS; ++r) ag[r] = au[r] = 0.f;
  for (int64_t cw = (int64_t)lane * CH; cw < C; cw += 64 * CH) {
    uint32_t gw[MV_ROWS][NW], uw[MV_ROWS][NW];
#pragma unroll
    for (int r = 0; r < MV_ROWS; ++r) {
      const int64_t row = row0 + r;
      if (row < a.I) {
        load_codes<16, CH>(gbase + row * C * 2, cw, gw[r]);
        load_codes<16, CH>(ubase + row * C * 2, cw, uw[r]);
      } else {
#pragma unroll
        for (int q = 0; q < NW; ++q) gw[r][q] = uw[r][q] = 0u;
      }
    }
    XChunk<XT, CH> xc;
    xc.load(xrow, cw);
    const int64_t g = cw / a.cpg_h;
#pragma unroll
    for (int r = 0; r < MV_ROWS; ++r) {
      const int64_t row = row0 + r;
      if (row < a.I) {
        const int64_t si = (e * a.I + row) * a.Gh + g;
        ag[r] += chunk_dot<16, XT, CH>(gw[r], tab, xc) * scale_at(a.gs, a.sdt, si);
        au[r] += chunk_dot<16, XT, CH>(uw[r], tab, xc) * scale_at(a.us, a.sdt, si);
      }
    }
  }
#pragma unroll
  for (int r = 0; r < MV_ROWS; ++r) {
    ag[r] = wave_sum(ag[r]);
    au[r] = wave_sum(au[r]);
  }
  if (lane < MV_ROWS && row0 + lane < a.I)
    hrow[row0 + lane] = from_float<bf16s>(swiglu(select_row(ag, lane), select_row(au, lane), a.limit));
}

// Down projection of every route of one token for MV_ROWS output rows, with
// the routing-weighted combine in fp32 (no atomics: one wave owns its rows).
// Reads the bf16 h of k_moe_gateup (bf16 codebook pairs, v_dot2_f32_bf16).
template <int CH>
__global__ __launch_bounds__(256) void k_moe_down(MoeArgs a) {
  using XT = bf16s;
  constexpr int NW = (CH * 2 + 3) / 4;
  constexpr int PK = PairOf<XT>::value;
  __shared__ uint4 tab[256];
  build_codebook<16, PK>(tab, a.table);
  __syncthreads();
  const int lane = threadIdx.x & 63;
  const int wv = threadIdx.x >> 6;
  const int64_t t = blockIdx.x / a.rb_d;
  const int64_t rb = blockIdx.x - t * a.rb_d;
  const int64_t row0 = (rb * MV_WAVES + wv) * MV_ROWS;
  if (row0 >= a.H) return;
  const int64_t C = a.I >> 3;
  float acc[MV_ROWS];
#pragma unroll
  for (int r = 0; r < MV_ROWS; ++r) acc[r] = 0.f;
  bool bad = false;
  for (int64_t j = 0; j < a.k; ++j) {
    const int64_t route = t * a.k + j;
    const float wt = a.w[route];
    if (wt == 0.f) continue;
    const int64_t e = a.idx[route];
    if (e < 0 || e >= a.E) {
      bad = true;
      continue;
    }
    const XT* hrow = (const XT*)a.h + route * a.I;
    const char* dbase = (const char*)a.dc + (e * a.H) * C * 2;
    float aj[MV_ROWS];
#pragma unroll
    for (int r = 0; r < MV_ROWS; ++r) aj[r] = 0.f;
    for (int64_t cw = (int64_t)lane * CH; cw < C; cw += 64 * CH) {
      uint32_t dw[MV_ROWS][NW];
#pragma unroll
      for (int r = 0; r < MV_ROWS; ++r) {
        const int64_t row = row0 + r;
        if (row < a.H) load_codes<16, CH>(dbase + row * C * 2, cw, dw[r]);
        else
#pragma unroll
          for (int q = 0; q < NW; ++q) dw[r][q] = 0u;
      }
      XChunk<XT, CH> xc;
      xc.load(hrow, cw);
      const int64_t g = cw / a.cpg_i;
#pragma unroll
      for (int r = 0; r < MV_ROWS; ++r) {
        const int64_t row = row0 + r;
        if (row < a.H) aj[r] += chunk_dot<16, XT, CH>(dw[r], tab, xc) * scale_at(a.ds, a.sdt, (e * a.H + row) * a.Gi + g);
      }
    }
#pragma unroll
    for (int r = 0; r < MV_ROWS; ++r) acc[r] = fmaf(wt, aj[r], acc[r]);
  }
#pragma unroll
  for (int r = 0; r < MV_ROWS; ++r) acc[r] = wave_sum(acc[r]);
  if (lane < MV_ROWS && row0 + lane < a.H)
    store_at(a.out, a.odt, t * a.H + row0 + lane, bad ? __builtin_nanf("") : select_row(acc, lane));
}

// ------------------------------------------------------------------ host side

// Codewords per lane chunk: must divide the codewords of a scale group (and of
// the residual's group) so a chunk never straddles two scales; prefer the
// widest load that keeps all 64 lanes busy.
static int pick_chunk(int64_t C, int64_t cpg, int64_t rcpg) {
  auto ok = [&](int ch) { return cpg % ch == 0 && (rcpg <= 0 || rcpg % ch == 0); };
  if (ok(8) && C % 512 == 0) return 8;
  if (ok(4) && C % 256 == 0) return 4;
  for (int ch : {8, 4, 2, 1})
    if (ok(ch) && C >= 64 * ch) return ch;
  for (int ch : {8, 4, 2, 1})
    if (ok(ch)) return ch;
  return 1;
}

template <int CB, typename XT, bool NESTED>
static void launch_matvec_ch(int ch, dim3 grid, hipStream_t s, const MatvecArgs& a) {
  switch (ch) {
    case 8: hipLaunchKernelGGL((k_vq_matvec<CB, XT, 8, NESTED>), grid, dim3(256), 0, s, a); break;
    case 4: hipLaunchKernelGGL((k_vq_matvec<CB, XT, 4, NESTED>), grid, dim3(256), 0, s, a); break;
    case 2: hipLaunchKernelGGL((k_vq_matvec<CB, XT, 2, NESTED>), grid, dim3(256), 0, s, a); break;
    default: hipLaunchKernelGGL((k_vq_matvec<CB, XT, 1, NESTED>), grid, dim3(256), 0, s, a); break;
  }
}

template <typename XT>
static void launch_matvec_x(int cb, bool nested, int ch, dim3 grid, hipStream_t s, const MatvecArgs& a) {
  if (cb == 8) launch_matvec_ch<8, XT, false>(ch, grid, s, a);
  else if (nested) launch_matvec_ch<16, XT, true>(ch, grid, s, a);
  else launch_matvec_ch<16, XT, false>(ch, grid, s, a);
}

}  // namespace keep

using namespace keep;

extern "C" int keep_e8p_decode(const uint16_t* codes, int64_t n, const uint32_t* table, const void* scales,
                               int scale_dtype, int64_t codewords_per_row, int64_t group_codewords, float* out,
                               void* stream) {
  KEEP_REQUIRE_DIMS(n, codewords_per_row, group_codewords);
  KEEP_REQUIRE(n >= 0, "n must be >= 0");
  if (n == 0) return KEEP_OK;
  KEEP_REQUIRE(codes && table && out, "codes, table and out must be non-null");
  KEEP_REQUIRE(aligned(out, 16), "out must be 16-byte aligned");
  if (scales) {
    KEEP_REQUIRE(dtype_ok(scale_dtype), "bad scale dtype %d", scale_dtype);
    KEEP_REQUIRE(codewords_per_row > 0 && n % codewords_per_row == 0, "n must be a multiple of codewords_per_row");
    KEEP_REQUIRE(group_codewords > 0 && codewords_per_row % group_codewords == 0,
                 "codewords_per_row must be a multiple of group_codewords");
  }
  int64_t blocks = (n + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  hipLaunchKernelGGL((k_e8p_decode<PAIR_F16>), dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream, codes, n,
                     table, scales, scale_dtype, codewords_per_row, group_codewords, out);
  return launch_status("keep_e8p_decode");
}

extern "C" int keep_e8_1bit_decode(const uint8_t* codes, int64_t n, const uint32_t* table, const void* scales,
                                   int scale_dtype, int64_t codewords_per_row, int64_t group_codewords, float* out,
                                   void* stream) {
  KEEP_REQUIRE_DIMS(n, codewords_per_row, group_codewords);
  KEEP_REQUIRE(n >= 0, "n must be >= 0");
  if (n == 0) return KEEP_OK;
  KEEP_REQUIRE(codes && table && out, "codes, table and out must be non-null");
  KEEP_REQUIRE(aligned(out, 16), "out must be 16-byte aligned");
  if (scales) {
    KEEP_REQUIRE(dtype_ok(scale_dtype), "bad scale dtype %d", scale_dtype);
    KEEP_REQUIRE(codewords_per_row > 0 && n % codewords_per_row == 0, "n must be a multiple of codewords_per_row");
    KEEP_REQUIRE(group_codewords > 0 && codewords_per_row % group_codewords == 0,
                 "codewords_per_row must be a multiple of group_codewords");
  }
  int64_t blocks = (n + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  hipLaunchKernelGGL(k_e8_decode, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream, codes, n, table, scales,
                     scale_dtype, codewords_per_row, group_codewords, out);
  return launch_status("keep_e8_1bit_decode");
}

extern "C" int keep_vq_matvec(const void* x, int x_dtype, int64_t x_rows, const void* codes, int code_bits,
                              const void* scales, int scale_dtype, const uint32_t* table, const int32_t* rhs,
                              const int32_t* lhs, int64_t routes, int64_t x_div, int64_t num_experts, int64_t N,
                              int64_t K, int64_t group_size, const uint8_t* res_codes, const void* res_scales,
                              int64_t res_group_size, const uint32_t* res_table, const uint32_t* hot_of_slot,
                              int64_t num_hot, void* out, int out_dtype, void* stream) {
  KEEP_REQUIRE_DIMS(x_rows, routes, x_div, num_experts, N, K, group_size, res_group_size, num_hot);
  KEEP_REQUIRE(code_bits == 8 || code_bits == 16, "code_bits must be 8 or 16, got %d", code_bits);
  KEEP_REQUIRE(dtype_ok(x_dtype) && dtype_ok(scale_dtype) && dtype_ok(out_dtype), "bad dtype enum");
  KEEP_REQUIRE(N > 0 && K > 0 && K % 8 == 0, "need N > 0 and K > 0 divisible by 8 (N=%lld K=%lld)", (long long)N,
               (long long)K);
  KEEP_REQUIRE(group_size > 0 && group_size % 8 == 0 && K % group_size == 0,
               "group_size must be a positive multiple of 8 dividing K (group_size=%lld)", (long long)group_size);
  KEEP_REQUIRE(routes >= 0 && num_experts > 0, "need routes >= 0 and num_experts > 0");
  if (routes == 0) return KEEP_OK;
  KEEP_REQUIRE(x && codes && scales && table && out, "null pointer argument");
  KEEP_REQUIRE(rhs || num_experts == 1, "rhs may be NULL only for one matrix (num_experts == 1)");
  KEEP_REQUIRE(lhs || x_div > 0, "x_div must be > 0 without lhs");
  KEEP_REQUIRE(x_rows > 0, "x_rows must be > 0");
  KEEP_REQUIRE(aligned(x, 16), "x must be 16-byte aligned");
  const bool nested = res_codes != nullptr;
  if (nested) {
    KEEP_REQUIRE(code_bits == 16, "a nested residual needs 16-bit base codes");
    KEEP_REQUIRE(res_scales && res_table && hot_of_slot && num_hot > 0, "nested residual needs scales, table, hot_of_slot");
    KEEP_REQUIRE(res_group_size > 0 && res_group_size % 8 == 0 && K % res_group_size == 0, "bad res_group_size");
  }
  const int64_t C = K / 8;
  const int64_t cpg = group_size / 8;
  const int64_t rcpg = nested ? res_group_size / 8 : 0;
  const int ch = pick_chunk(C, cpg, rcpg);
  KEEP_REQUIRE(aligned(codes, (uintptr_t)(ch * code_bits / 8)), "codes pointer misaligned for %d-codeword loads", ch);
  if (nested) KEEP_REQUIRE(aligned(res_codes, (uintptr_t)ch), "res_codes misaligned");
  MatvecArgs a{};
  a.x = x; a.x_rows = x_rows; a.codes = codes; a.scales = scales; a.sdt = scale_dtype; a.table = table;
  a.rhs = rhs; a.lhs = lhs; a.routes = routes; a.x_div = x_div > 0 ? x_div : 1;
  a.E = num_experts; a.N = N; a.K = K; a.G = K / group_size; a.cpg = cpg;
  a.rcodes = res_codes; a.rscales = res_scales; a.rG = nested ? K / res_group_size : 1; a.rcpg = nested ? rcpg : 1;
  a.rtable = res_table; a.hot = hot_of_slot; a.nhot = num_hot; a.out = out; a.odt = out_dtype;
  a.row_blocks = (N + MV_WAVES * MV_ROWS - 1) / (MV_WAVES * MV_ROWS);
  const int64_t blocks = a.row_blocks * routes;
  KEEP_REQUIRE(blocks <= 0x7fffffffLL, "too many blocks");
  dim3 grid((unsigned)blocks);
  hipStream_t s = (hipStream_t)stream;
  if (x_dtype == KEEP_F16) launch_matvec_x<_Float16>(code_bits, nested, ch, grid, s, a);
  else if (x_dtype == KEEP_BF16) launch_matvec_x<bf16s>(code_bits, nested, ch, grid, s, a);
  else launch_matvec_x<float>(code_bits, nested, ch, grid, s, a);
  return launch_status("keep_vq_matvec");
}

template <int CB, typename XT>
static void launch_tiles_cb(int ch, dim3 grid, hipStream_t s, const TileArgs& a) {
  switch (ch) {
    case 8: hipLaunchKernelGGL((k_vq_matvec_tiles<CB, XT, 8>), grid, dim3(256), 0, s, a); break;
    case 4: hipLaunchKernelGGL((k_vq_matvec_tiles<CB, XT, 4>), grid, dim3(256), 0, s, a); break;
    case 2: hipLaunchKernelGGL((k_vq_matvec_tiles<CB, XT, 2>), grid, dim3(256), 0, s, a); break;
    default: hipLaunchKernelGGL((k_vq_matvec_tiles<CB, XT, 1>), grid, dim3(256), 0, s, a); break;
  }
}
template <typename XT>
static void launch_tiles(int code_bits, int ch, dim3 grid, hipStream_t s, const TileArgs& a) {
  if (code_bits == 16) launch_tiles_cb<16, XT>(ch, grid, s, a);
  else launch_tiles_cb<8, XT>(ch, grid, s, a);
}

extern "C" int keep_vq_matvec_tiles(const void* x, int x_dtype, int64_t x_rows, const void* codes, int code_bits,
                                    const void* scales, int scale_dtype, const uint32_t* table,
                                    const int32_t* sorted_lhs, int64_t routes, const int32_t* tile_expert,
                                    const int32_t* tile_offset, const int32_t* tile_count, int64_t n_tiles,
                                    int64_t m_rows, int64_t num_experts, int64_t N, int64_t K, int64_t group_size,
                                    void* out, int out_dtype, void* stream) {
  KEEP_REQUIRE_DIMS(x_rows, routes, n_tiles, m_rows, num_experts, N, K, group_size);
  KEEP_REQUIRE(dtype_ok(x_dtype) && dtype_ok(scale_dtype) && dtype_ok(out_dtype), "bad dtype enum");
  KEEP_REQUIRE(code_bits == 8 || code_bits == 16, "code_bits must be 8 or 16, got %d", code_bits);
  KEEP_REQUIRE(N > 0 && K > 0 && K % 8 == 0, "need N > 0 and K divisible by 8");
  KEEP_REQUIRE(group_size > 0 && group_size % 8 == 0 && K % group_size == 0, "bad group_size");
  KEEP_REQUIRE(m_rows >= 1 && m_rows <= 8, "m_rows must be in 1..8, got %lld", (long long)m_rows);
  KEEP_REQUIRE(n_tiles >= 0 && routes >= 0, "negative sizes");
  if (n_tiles == 0 || routes == 0) return KEEP_OK;
  KEEP_REQUIRE(x && codes && scales && table && sorted_lhs && tile_expert && tile_offset && tile_count && out,
               "null pointer argument");
  KEEP_REQUIRE(x_rows > 0 && aligned(x, 16), "x must be non-empty and 16-byte aligned");
  const int64_t C = K / 8, cpg = group_size / 8;
  const int ch = pick_chunk(C, cpg, 0);
  KEEP_REQUIRE(aligned(codes, (uintptr_t)(ch * code_bits / 8)), "codes misaligned");
  TileArgs a{};
  a.x = x; a.x_rows = x_rows; a.codes = codes; a.scales = scales; a.sdt = scale_dtype; a.table = table;
  a.lhs = sorted_lhs; a.routes = routes; a.te = tile_expert; a.to = tile_offset; a.tc = tile_count;
  a.n_tiles = n_tiles; a.m_rows = m_rows; a.E = num_experts; a.N = N; a.K = K; a.G = K / group_size; a.cpg = cpg;
  a.out = out; a.odt = out_dtype;
  a.row_blocks = (N + MV_WAVES * MV_ROWS - 1) / (MV_WAVES * MV_ROWS);
  const int64_t blocks = a.row_blocks * n_tiles;
  KEEP_REQUIRE(blocks <= 0x7fffffffLL, "too many blocks");
  dim3 grid((unsigned)blocks);
  hipStream_t s = (hipStream_t)stream;
  if (x_dtype == KEEP_F16) launch_tiles<_Float16>(code_bits, ch, grid, s, a);
  else if (x_dtype == KEEP_BF16) launch_tiles<bf16s>(code_bits, ch, grid, s, a);
  else launch_tiles<float>(code_bits, ch, grid, s, a);
  return launch_status("keep_vq_matvec_tiles");
}

template <typename XT>
static void launch_moe(int ch_h, int ch_i, bool gateup, bool down, hipStream_t s, const MoeArgs& a) {
  dim3 g1((unsigned)(a.rb_gu * a.T * a.k)), g2((unsigned)(a.rb_d * a.T));
  if (gateup) {
    switch (ch_h) {
      case 8: hipLaunchKernelGGL((k_moe_gateup<XT, 8>), g1, dim3(256), 0, s, a); break;
      case 4: hipLaunchKernelGGL((k_moe_gateup<XT, 4>), g1, dim3(256), 0, s, a); break;
      case 2: hipLaunchKernelGGL((k_moe_gateup<XT, 2>), g1, dim3(256), 0, s, a); break;
      default: hipLaunchKernelGGL((k_moe_gateup<XT, 1>), g1, dim3(256), 0, s, a); break;
    }
  }
  if (down) {
    switch (ch_i) {
      case 8: hipLaunchKernelGGL((k_moe_down<8>), g2, dim3(256), 0, s, a); break;
      case 4: hipLaunchKernelGGL((k_moe_down<4>), g2, dim3(256), 0, s, a); break;
      case 2: hipLaunchKernelGGL((k_moe_down<2>), g2, dim3(256), 0, s, a); break;
      default: hipLaunchKernelGGL((k_moe_down<1>), g2, dim3(256), 0, s, a); break;
    }
  }
}

static int moe_common(bool gateup, bool down, const char* what, const void* x, int x_dtype, int64_t T, int64_t H,
                      int64_t I, const int32_t* idx, const float* w, int64_t k, int64_t num_experts,
                      const uint16_t* gate_codes, const void* gate_scales, const uint16_t* up_codes,
                      const void* up_scales, const uint16_t* down_codes, const void* down_scales, int scale_dtype,
                      int64_t group_size_h, int64_t group_size_i, const uint32_t* table, const void* prepared,
                      float swiglu_limit, void* h_work, void* out, int out_dtype, void* stream) {
  KEEP_REQUIRE(gateup ? (x_dtype == KEEP_F16 || x_dtype == KEEP_BF16) : x_dtype == KEEP_BF16,
               gateup ? "fused MoE needs fp16 or bf16 activations" : "h_work must be bf16 (h_dtype = KEEP_BF16)");
  KEEP_REQUIRE(dtype_ok(scale_dtype) && dtype_ok(out_dtype), "bad dtype enum");
  KEEP_REQUIRE(T >= 0 && k > 0 && num_experts > 0, "need T >= 0, k > 0, num_experts > 0");
  KEEP_REQUIRE(H > 0 && I > 0 && H % 8 == 0 && I % 8 == 0, "H and I must be positive multiples of 8");
  KEEP_REQUIRE(group_size_h > 0 && group_size_h % 8 == 0 && H % group_size_h == 0, "bad group_size_h");
  KEEP_REQUIRE(group_size_i > 0 && group_size_i % 8 == 0 && I % group_size_i == 0, "bad group_size_i");
  if (T == 0) return KEEP_OK;
  KEEP_REQUIRE(idx && w && table && h_work, "null pointer argument");
  KEEP_REQUIRE(!gateup || (x && gate_codes && gate_scales && up_codes && up_scales), "null gate/up argument");
  KEEP_REQUIRE(!down || (down_codes && down_scales && out), "null down argument");
  KEEP_REQUIRE((!x || aligned(x, 16)) && aligned(h_work, 16), "x and h_work must be 16-byte aligned");
  const int ch_h = pick_chunk(H / 8, group_size_h / 8, 0);
  const int ch_i = pick_chunk(I / 8, group_size_i / 8, 0);
  KEEP_REQUIRE((!gateup || (aligned(gate_codes, ch_h * 2) && aligned(up_codes, ch_h * 2))) &&
                   (!down || aligned(down_codes, ch_i * 2)),
               "codes misaligned");
  (void)prepared;
  MoeArgs a{};
  a.x = x; a.T = T; a.H = H; a.I = I; a.idx = idx; a.w = w; a.k = k; a.E = num_experts;
  a.gc = gate_codes; a.uc = up_codes; a.dc = down_codes; a.gs = gate_scales; a.us = up_scales; a.ds = down_scales;
  a.sdt = scale_dtype; a.Gh = H / group_size_h; a.cpg_h = group_size_h / 8; a.Gi = I / group_size_i;
  a.cpg_i = group_size_i / 8; a.table = table; a.limit = swiglu_limit; a.h = h_work; a.out = out; a.odt = out_dtype;
  a.rb_gu = (I + MV_WAVES * MV_ROWS - 1) / (MV_WAVES * MV_ROWS);
  a.rb_d = (H + MV_WAVES * MV_ROWS - 1) / (MV_WAVES * MV_ROWS);
  KEEP_REQUIRE(T * k <= 0x7fffffffLL && a.rb_gu * (T * k) <= 0x7fffffffLL && a.rb_d * T <= 0x7fffffffLL,
               "too many blocks");
  hipStream_t s = (hipStream_t)stream;
  if (x_dtype == KEEP_F16) launch_moe<_Float16>(ch_h, ch_i, gateup, down, s, a);
  else launch_moe<bf16s>(ch_h, ch_i, gateup, down, s, a);
  return launch_status(what);
}

extern "C" int keep_moe_decode(const void* x, int x_dtype, int64_t T, int64_t H, int64_t I, const int32_t* idx,
                               const float* w, int64_t k, int64_t num_experts, const uint16_t* gate_codes,
                               const void* gate_scales, const uint16_t* up_codes, const void* up_scales,
                               const uint16_t* down_codes, const void* down_scales, int scale_dtype,
                               int64_t group_size_h, int64_t group_size_i, const uint32_t* table,
                               const void* prepared, float swiglu_limit, void* h_work, void* out, int out_dtype,
                               void* stream) {
  KEEP_REQUIRE_DIMS(T, H, I, k, num_experts, group_size_h, group_size_i);
  return moe_common(true, true, "keep_moe_decode", x, x_dtype, T, H, I, idx, w, k, num_experts, gate_codes,
                    gate_scales, up_codes, up_scales, down_codes, down_scales, scale_dtype, group_size_h,
                    group_size_i, table, prepared, swiglu_limit, h_work, out, out_dtype, stream);
}

extern "C" int keep_moe_gateup(const void* x, int x_dtype, int64_t T, int64_t H, int64_t I, const int32_t* idx,
                               const float* w, int64_t k, int64_t num_experts, const uint16_t* gate_codes,
                               const void* gate_scales, const uint16_t* up_codes, const void* up_scales,
                               int scale_dtype, int64_t group_size_h, const uint32_t* table, const void* prepared,
                               float swiglu_limit, void* h_work, void* stream) {
  KEEP_REQUIRE_DIMS(T, H, I, k, num_experts, group_size_h);
  return moe_common(true, false, "keep_moe_gateup", x, x_dtype, T, H, I, idx, w, k, num_experts, gate_codes,
                    gate_scales, up_codes, up_scales, nullptr, nullptr, scale_dtype, group_size_h, I, table,
                    prepared, swiglu_limit, h_work, nullptr, KEEP_F32, stream);
}

extern "C" int keep_moe_down(int h_dtype, int64_t T, int64_t H, int64_t I, const int32_t* idx, const float* w,
                             int64_t k, int64_t num_experts, const uint16_t* down_codes, const void* down_scales,
                             int scale_dtype, int64_t group_size_i, const uint32_t* table, const void* prepared,
                             const void* h_work, void* out, int out_dtype, void* stream) {
  KEEP_REQUIRE_DIMS(T, H, I, k, num_experts, group_size_i);
  return moe_common(false, true, "keep_moe_down", nullptr, h_dtype, T, H, I, idx, w, k, num_experts, nullptr,
                    nullptr, nullptr, nullptr, down_codes, down_scales, scale_dtype, H, group_size_i, table,
                    prepared, 0.f, const_cast<void*>(h_work), out, out_dtype, stream);
}

extern "C" int keep_e8_1bit_matvec(const void* x, int x_dtype, int64_t x_rows, const uint8_t* codes,
                                   const void* scales, int scale_dtype, const uint32_t* table, const uint32_t* rhs,
                                   int64_t routes, int64_t x_div, int64_t num_experts, int64_t N, int64_t K,
                                   int64_t group_size, void* out, int out_dtype, void* stream) {
  KEEP_REQUIRE_DIMS(x_rows, routes, x_div, num_experts, N, K, group_size);
  KEEP_REQUIRE(dtype_ok(x_dtype) && dtype_ok(scale_dtype) && dtype_ok(out_dtype), "bad dtype enum");
  KEEP_REQUIRE(N > 0 && K > 0 && K % 8 == 0, "need N > 0 and K > 0 divisible by 8 (N=%lld K=%lld)", (long long)N,
               (long long)K);
  KEEP_REQUIRE(group_size > 0 && group_size % 8 == 0 && K % group_size == 0,
               "group_size must be a positive multiple of 8 dividing K (group_size=%lld)", (long long)group_size);
  KEEP_REQUIRE(routes >= 0 && num_experts > 0 && x_div > 0, "need routes >= 0, num_experts > 0 and x_div > 0");
  if (routes == 0) return KEEP_OK;
  KEEP_REQUIRE(x && codes && scales && table && rhs && out, "null pointer argument");
  KEEP_REQUIRE(x_rows > 0 && aligned(x, 16), "x must be non-empty and 16-byte aligned");
  const int64_t C = K / 8, cpg = group_size / 8;
  const int ch = pick_chunk(C, cpg, 0);
  KEEP_REQUIRE(aligned(codes, (uintptr_t)ch), "codes pointer misaligned for %d-codeword loads", ch);
  MatvecArgs a{};
  a.x = x; a.x_rows = x_rows; a.codes = codes; a.scales = scales; a.sdt = scale_dtype; a.table = table;
  a.rhs = (const int32_t*)rhs; a.lhs = nullptr; a.routes = routes; a.x_div = x_div;
  a.E = num_experts; a.N = N; a.K = K; a.G = K / group_size; a.cpg = cpg; a.rG = 1; a.rcpg = 1;
  a.out = out; a.odt = out_dtype; a.zero_none = 1;
  a.row_blocks = (N + MV_WAVES * MV_ROWS - 1) / (MV_WAVES * MV_ROWS);
  const int64_t blocks = a.row_blocks * routes;
  KEEP_REQUIRE(blocks <= 0x7fffffffLL, "too many blocks");
  dim3 grid((unsigned)blocks);
  hipStream_t s = (hipStream_t)stream;
  if (x_dtype == KEEP_F16) launch_matvec_x<_Float16>(8, false, ch, grid, s, a);
  else if (x_dtype == KEEP_BF16) launch_matvec_x<bf16s>(8, false, ch, grid, s, a);
  else launch_matvec_x<float>(8, false, ch, grid, s, a);
  return launch_status("keep_e8_1bit_matvec");
}
