// Prefill grouped GEMM over expert-sorted routes on gfx950 MFMA
// (v_mfma_f32_32x32x16_{f16,bf16}).
//
// Block = 4 waves = one route tile (<= 64 routes of one expert: two 32-route
// m-tiles) x 256 weight rows (each wave: 64 rows = two 32-row n-tiles).
// Out[m, n] = sum_k X[lhs[m], k] W[n, k], i.e. MFMA A = gathered activations
// (M x K), B = decoded weights (K x N).
//
// No LDS weight tile: in the 32x32x16 operand layout lane l holds 8
// consecutive k of one B column (n = l % 32) -- exactly one E8P codeword of
// row n -- so each lane decodes its codeword straight into the B operand
// registers (LDS codebook lookup + sign XOR + the +-1/4 shift as a packed
// add; every value is exact in fp16/bf16). The k order inside a K block is
// permuted so a lane's 8 codewords are contiguous (one 16-byte load): lane
// half h = l / 32 takes codewords [8h, 8h + 8) of a 128-wide K block, and at
// k-step s uses codeword 8h + s; the A operand reads the same k range.
// Activations are gathered through lhs inside the kernel (no sorted copy).
// Scales: one fp32 multiply per (row, group) -- per-group partial
// accumulators are folded into the total at each group boundary.
//
// Tile -> block mapping is XCD-aware: logical work item w = nblk * n_tiles +
// tile (tiles of one expert adjacent) is placed so that consecutive w run on
// the same XCD, keeping an expert's code rows in that XCD's L2 while its
// route tiles are processed.
#include "common.h"

namespace keep {

typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf8_t __attribute__((ext_vector_type(8)));
typedef float f16v_t __attribute__((ext_vector_type(16)));

constexpr int GM_WAVES = 4;
constexpr int GM_NB = 256;  // weight rows per block
constexpr int GM_KB = 128;  // k per K block (16 codewords)
constexpr int GM_XCDS = 8;

struct GemmArgs {
  const void* x;
  int64_t x_rows;
  const int32_t* lhs;
  const uint16_t* codes;
  const void* scales;
  int sdt;
  const uint32_t* table;
  const int32_t *te, *to, *tc;
  int64_t n_tiles, routes;
  int64_t E, N, K, G, cpg;
  void* out;
  int odt;
  int64_t nblocks_n, total, per_xcd;
};

__device__ __forceinline__ float gm_scale(const void* p, int dt, int64_t i) {
  if (dt == KEEP_F16) return (float)((const _Float16*)p)[i];
  if (dt == KEEP_BF16) return __uint_as_float((uint32_t)((const uint16_t*)p)[i] << 16);
  return ((const float*)p)[i];
}

__device__ __forceinline__ void gm_store(void* p, int dt, int64_t i, float v) {
  if (dt == KEEP_F16) ((_Float16*)p)[i] = (_Float16)v;
  else if (dt == KEEP_BF16) ((uint16_t*)p)[i] = from_float<bf16s>(v).bits;
  else ((float*)p)[i] = v;
}

template <int PK>
__device__ __forceinline__ uint32_t add_shift(uint32_t w, float shift) {
  if constexpr (PK == PAIR_F16) {
    h2_t v = __builtin_bit_cast(h2_t, w);
    const _Float16 s = (_Float16)shift;
    v = v + h2_t{s, s};
    return __builtin_bit_cast(uint32_t, v);
  } else {
    const float lo = __uint_as_float(w << 16) + shift;
    const float hi = __uint_as_float(w & 0xffff0000u) + shift;
    return (__float_as_uint(lo) >> 16) | (__float_as_uint(hi) & 0xffff0000u);  // exact
  }
}

// Decode codeword c into the 8 B-operand elements (4 packed pairs).
template <int PK>
__device__ __forceinline__ uint4 decode_operand(uint32_t c, const uint4* tab) {
  const E8PSigns sg = e8p_signs(c);
  const uint4 e = tab[(c >> 8) & 0xffu];
  return make_uint4(add_shift<PK>(e.x ^ sg.m0, sg.shift), add_shift<PK>(e.y ^ sg.m1, sg.shift),
                    add_shift<PK>(e.z ^ sg.m2, sg.shift), add_shift<PK>(e.w ^ sg.m3, sg.shift));
}

template <int PK>
__device__ __forceinline__ f16v_t mfma(uint4 a, uint4 b, f16v_t c) {
  if constexpr (PK == PAIR_F16) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(h8_t, a), __builtin_bit_cast(h8_t, b), c, 0, 0,
                                                  0);
  } else {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf8_t, a), __builtin_bit_cast(bf8_t, b), c, 0,
                                                   0, 0);
  }
}

template <int PK, bool GROUPED>
__global__ __launch_bounds__(256) void k_grouped_gemm(GemmArgs a) {
  __shared__ uint4 tab[256];
  build_codebook<16, PK>(tab, a.table);
  __syncthreads();
  const int64_t b = blockIdx.x;
  const int64_t w = (b % GM_XCDS) * a.per_xcd + b / GM_XCDS;
  if (w >= a.total) return;
  const int64_t nblk = w / a.n_tiles;
  const int64_t tile = w - nblk * a.n_tiles;
  const int cnt_raw = a.tc[tile];
  if (cnt_raw <= 0) return;
  const int cnt = cnt_raw < 64 ? cnt_raw : 64;
  const int64_t off = a.to[tile];
  const int64_t e = a.te[tile];
  if (off < 0 || off + cnt > a.routes) return;  // nothing can be written safely
  const int lane = threadIdx.x & 63;
  const int wv = threadIdx.x >> 6;
  const int h = lane >> 5;
  const int l32 = lane & 31;
  const int64_t n0 = nblk * GM_NB + wv * 64;
  if (n0 >= a.N) return;
  const bool bad = e < 0 || e >= a.E || cnt_raw > 64;  // written as NaN rows
  const int64_t C = a.K >> 3;

  // activation rows of this lane's two m positions
  int64_t xrow[2];
  bool xbad = bad;
#pragma unroll
  for (int mt = 0; mt < 2; ++mt) {
    const int m = mt * 32 + l32;
    const int mm = m < cnt ? m : 0;
    int64_t r = bad ? 0 : (a.lhs ? (int64_t)a.lhs[off + mm] : off + mm);
    if (r < 0 || r >= a.x_rows) {
      if (m < cnt) xbad = true;
      r = 0;
    }
    xrow[mt] = r;
  }
  const uint16_t* xb = (const uint16_t*)a.x;
  // code rows of this lane's two n positions
  const uint16_t* crow[2];
  bool nvalid[2];
#pragma unroll
  for (int nt = 0; nt < 2; ++nt) {
    const int64_t n = n0 + nt * 32 + l32;
    nvalid[nt] = n < a.N && !bad;
    crow[nt] = a.codes + ((nvalid[nt] ? e * a.N + n : 0) * C);
  }

  f16v_t acc[2][2], part[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      acc[i][j] = f16v_t{};
      part[i][j] = f16v_t{};
    }

  const int64_t nkb = a.K / GM_KB;
  const int64_t kb_per_group = a.cpg / 16;
  for (int64_t kb = 0; kb < nkb; ++kb) {
    const int64_t cw0 = kb * 16 + 8 * h;  // this lane's first codeword of the block
    uint4 cw[2];
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) cw[nt] = nvalid[nt] ? *(const uint4*)(crow[nt] + cw0) : make_uint4(0, 0, 0, 0);
    uint4 xa[2][8];
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
      const uint4* p = (const uint4*)(xb + xrow[mt] * a.K + cw0 * 8);
#pragma unroll
      for (int s = 0; s < 8; ++s) xa[mt][s] = p[s];
    }
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      uint4 bop[2];
#pragma unroll
      for (int nt = 0; nt < 2; ++nt) {
        const uint32_t word = (&cw[nt].x)[s >> 1];
        const uint32_t c = (s & 1) ? (word >> 16) : (word & 0xffffu);
        bop[nt] = decode_operand<PK>(c, tab);
      }
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) {
          if constexpr (GROUPED) part[mt][nt] = mfma<PK>(xa[mt][s], bop[nt], part[mt][nt]);
          else acc[mt][nt] = mfma<PK>(xa[mt][s], bop[nt], acc[mt][nt]);
        }
    }
    if constexpr (GROUPED) {
      if ((kb + 1) % kb_per_group == 0) {
        const int64_t g = kb / kb_per_group;
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) {
          const int64_t n = n0 + nt * 32 + l32;
          const float sc = nvalid[nt] ? gm_scale(a.scales, a.sdt, (e * a.N + n) * a.G + g) : 0.f;
#pragma unroll
          for (int mt = 0; mt < 2; ++mt) {
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[mt][nt][v] = fmaf(sc, part[mt][nt][v], acc[mt][nt][v]);
            part[mt][nt] = f16v_t{};
          }
        }
      }
    }
  }
  // epilogue
#pragma unroll
  for (int nt = 0; nt < 2; ++nt) {
    const int64_t n = n0 + nt * 32 + l32;
    if (n >= a.N) continue;
    float sc = 1.f;
    if constexpr (!GROUPED) sc = bad ? 0.f : gm_scale(a.scales, a.sdt, (e * a.N + n));
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int m = mt * 32 + 8 * (v >> 2) + 4 * h + (v & 3);
        if (m < cnt) {
          float val = acc[mt][nt][v];
          if constexpr (!GROUPED) val *= sc;
          if (bad || xbad) val = __builtin_nanf("");
          gm_store(a.out, a.odt, (off + m) * a.N + n, val);
        }
      }
  }
}

}  // namespace keep

using namespace keep;

extern "C" int keep_vq_grouped_gemm(const void* x, int x_dtype, int64_t x_rows, const int32_t* lhs,
                                    const uint16_t* codes, const void* scales, int scale_dtype, const uint32_t* table,
                                    const int32_t* tile_expert, const int32_t* tile_offset, const int32_t* tile_count,
                                    int64_t n_tiles, int64_t routes, int64_t num_experts, int64_t N, int64_t K,
                                    int64_t group_size, void* out, int out_dtype, void* stream) {
  KEEP_REQUIRE(x_dtype == KEEP_F16 || x_dtype == KEEP_BF16, "grouped GEMM needs fp16 or bf16 activations");
  KEEP_REQUIRE(dtype_ok(scale_dtype) && dtype_ok(out_dtype), "bad dtype enum");
  KEEP_REQUIRE(N > 0 && K > 0 && K % GM_KB == 0, "grouped GEMM needs K divisible by %d (K=%lld)", GM_KB,
               (long long)K);
  KEEP_REQUIRE(group_size > 0 && K % group_size == 0 && group_size % GM_KB == 0,
               "grouped GEMM needs group_size a multiple of %d dividing K (group_size=%lld)", GM_KB,
               (long long)group_size);
  KEEP_REQUIRE(n_tiles >= 0 && routes >= 0 && num_experts > 0, "bad sizes");
  if (n_tiles == 0 || routes == 0) return KEEP_OK;
  KEEP_REQUIRE(x && codes && scales && table && tile_expert && tile_offset && tile_count && out,
               "null pointer argument");
  KEEP_REQUIRE(x_rows > 0 && aligned(x, 16) && aligned(codes, 16), "x and codes must be 16-byte aligned");
  GemmArgs a{};
  a.x = x; a.x_rows = x_rows; a.lhs = lhs; a.codes = codes; a.scales = scales; a.sdt = scale_dtype; a.table = table;
  a.te = tile_expert; a.to = tile_offset; a.tc = tile_count; a.n_tiles = n_tiles; a.routes = routes;
  a.E = num_experts; a.N = N; a.K = K; a.G = K / group_size; a.cpg = group_size / 8; a.out = out; a.odt = out_dtype;
  a.nblocks_n = (N + GM_NB - 1) / GM_NB;
  a.total = a.nblocks_n * n_tiles;
  a.per_xcd = (a.total + GM_XCDS - 1) / GM_XCDS;
  const int64_t blocks = a.per_xcd * GM_XCDS;
  KEEP_REQUIRE(blocks <= 0x7fffffffLL, "too many blocks");
  const bool grouped = a.G > 1;
  hipStream_t s = (hipStream_t)stream;
  dim3 grid((unsigned)blocks);
  if (x_dtype == KEEP_F16) {
    if (grouped) hipLaunchKernelGGL((k_grouped_gemm<PAIR_F16, true>), grid, dim3(256), 0, s, a);
    else hipLaunchKernelGGL((k_grouped_gemm<PAIR_F16, false>), grid, dim3(256), 0, s, a);
  } else {
    if (grouped) hipLaunchKernelGGL((k_grouped_gemm<PAIR_BF16, true>), grid, dim3(256), 0, s, a);
    else hipLaunchKernelGGL((k_grouped_gemm<PAIR_BF16, false>), grid, dim3(256), 0, s, a);
  }
  return launch_status("keep_vq_grouped_gemm");
}
