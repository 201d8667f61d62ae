// Prefill grouped GEMM over expert-sorted routes on the fp16 matrix cores
// (v_mfma_f32_32x32x16_f16), for tiles of up to 64 routes of one expert (the
// sorted-route prefill of src/ramp/ops/vq_switch.py:286-377 and
// glm4_moe_adapter.py:274-353: one route plan shared by gate, up and down).
//
// Arithmetic. As the reference's sorted path (vq_switch.py:712-715,759-771:
// the gathered rows cast to float16, then an fp16 matmul), the A rows are fp16:
// fp16 rows as they are; bf16 and fp32 rows times a power of two r per row
// (k_gq_rowscale: max |x| r in [2^14, 2^15), so no row overflows fp16 and a
// bf16 row converts exactly), rounded to nearest even. B is the decoded weight
// x 4, an odd integer |q| <= 15 (E8P) or an even one in [-16, 14] (the nested
// tier's 8-bit E8), exact in fp16; products are exact in fp32 and the MFMA sums
// them in fp32. D / (4 r) x the column's scale is the output.
//
// B decode. The block's 64 KiB LDS image (built from T and M of
// keep_e8p_prepare, in natural dim order, T with every byte XOR 0x80) gives a
// codeword's 8 bytes q + 128 (mod 256) as T' ^ M in two 8-byte lookups (the
// decode-layer lookup addresses of q8_dev.h). A byte b becomes fp16 by placing
// it under the byte 0x64 (fp16 1024 + b) and subtracting 1152: four byte
// permutes and four packed fp16 adds per codeword.
//
// Layout. A 32x32x16 MFMA takes 8 k of one row (A) / column (B) per lane:
// lane half h = l / 32 at k-step s of a 128-wide K block takes codeword 8 h + s
// (the permutation of K within the block is the same for A and B), so a lane's
// codes for a K block are 8 consecutive codewords (one 16-byte load) and its A
// bytes at k-step s are row bytes 128 h + 16 s of the block. D element v of lane
// l is row 8 (v / 4) + 4 h + v % 4, column l % 32.
//
// Block = 8 waves, one work item = (route tile, 512 output columns); wave w
// owns 64 columns as two 32-column n-tiles and both 32-route m-tiles (the second
// is skipped when the tile holds <= 32 routes): each A operand read from LDS
// feeds two MFMAs. (Problems with fewer than four such items per CU take items
// of 256 columns, one n-tile per wave, to spread over the CUs.) The gate/up form pairs 16 gate rows with the same 16 up rows
// in each n-tile, so lanes l and l ^ 16 hold gate and up of one (route, row)
// and SwiGLU runs in the epilogue; h is written once, in bf16, at the route's
// sorted position.
//
// Pipeline. Persistent blocks (the LDS image is built once per block); a work
// item streams its K blocks with D blocks' code loads and A rows in flight in
// registers (every load unconditional and clamped at the end), the A rows of
// the next block staged into a second LDS buffer while the current one feeds
// the MFMAs; each k-step's image lookups are issued two k-steps ahead of its
// MFMAs and converted to fp16 one k-step ahead.
// Work items are spread XCD-aware (see the item loop).
#include <cstdlib>
#include <type_traits>

#include "common.h"
#include "moe_dev.h"
#include "q8_dev.h"

namespace keep {

constexpr int GQ_WAVES = 8;
constexpr int GQ_THREADS = 64 * GQ_WAVES;
constexpr int GQ_M = 64;                // routes per tile (two 32-row m-tiles)
constexpr int GQ_KB = 128;              // k per K block
constexpr int GQ_ROW = 2 * GQ_KB + 16;  // LDS bytes per A row: rows 4 banks apart (no conflicts)
constexpr int GQ_XCDS = 8;

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h2v __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

__device__ __forceinline__ f32x16 mfma32_f16(h8 a, h8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// Bytes q + 128 (mod 256) of eight integer weights q -> the fp16 values q.
__device__ __forceinline__ h8 gq_f16_of_bytes(uint2 b) {
  const uint32_t k = 0x64646464u;
  const uint32_t d[4] = {__builtin_amdgcn_perm(k, b.x, 0x04010400u), __builtin_amdgcn_perm(k, b.x, 0x04030402u),
                         __builtin_amdgcn_perm(k, b.y, 0x04010400u), __builtin_amdgcn_perm(k, b.y, 0x04030402u)};
  h8 r;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const h2v v = __builtin_bit_cast(h2v, d[i]) - h2v{(_Float16)1152.f, (_Float16)1152.f};
    r[2 * i] = v[0];
    r[2 * i + 1] = v[1];
  }
  return r;
}

// Natural-order bytes of a packed-nibble-order pair (dims 0, 2, 4, 6 | 1, 3, 5, 7).
__device__ __forceinline__ uint2 gq_natural(uint2 v) {
  return make_uint2(__builtin_amdgcn_perm(v.y, v.x, 0x05010400u), __builtin_amdgcn_perm(v.y, v.x, 0x07030602u));
}

// ------------------------------------------------------------------ row scales

// One wave per row: r = 2^(14 - floor(log2 max |x|)) (1 for a zero row, NaN for a
// row holding NaN or inf, which then reaches the row's outputs) and 1 / r.
template <typename XT>
__global__ __launch_bounds__(256) void k_gq_rowscale(const XT* x, int64_t rows, int K, float2* rs) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const XT* xr = x + row * K;
  float mx = 0.f;
  bool bad = false;
  for (int i = lane * 4; i < K; i += 256) {
    float v[4];
    if constexpr (sizeof(XT) == 4) {
      const float4 p = *(const float4*)(xr + i);
      v[0] = p.x; v[1] = p.y; v[2] = p.z; v[3] = p.w;
    } else {
      const uint2 p = *(const uint2*)(xr + i);
      v[0] = __uint_as_float(p.x << 16); v[1] = __uint_as_float(p.x & 0xffff0000u);
      v[2] = __uint_as_float(p.y << 16); v[3] = __uint_as_float(p.y & 0xffff0000u);
    }
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      bad |= !(fabsf(v[t]) <= 3.4028235e38f);  // NaN or inf
      mx = fmaxf(mx, fabsf(v[t]));
    }
  }
  mx = wave_max(mx);
  bad = __any(bad);
  if (lane == 0) {
    float r = 1.f, ri = 1.f;
    if (bad) {
      r = ri = __builtin_nanf("");
    } else if (mx > 0.f) {
      const int e = (int)((__float_as_uint(mx) >> 23) & 0xffu) - 127;  // floor(log2 mx) for a normal mx
      const int k = min(max(14 - e, -126), 127);
      r = __uint_as_float((uint32_t)(127 + k) << 23);
      ri = __uint_as_float((uint32_t)(127 - k) << 23);
    }
    rs[row] = make_float2(r, ri);
  }
}

// ------------------------------------------------------------------ grouped GEMM

struct GQArgs {
  const void* x;        // A rows [x_rows][K], fp16 / bf16 / fp32
  int xdt;
  const float2* rs;     // per A row (r, 1 / r) for bf16 / fp32 rows (null: fp16, r = 1)
  int64_t x_rows;
  const int32_t* lhs;   // sorted position -> A row (null: the position itself)
  const int32_t* oidx;  // sorted position -> output row (null: the position itself)
  const uint16_t *c0, *c1;  // codes [E][N][K / 8] (gate/up: gate, up)
  const void *s0, *s1;      // scales [E][N][G]
  int sdt;
  const void* tq;           // E8P: T and M (keep_e8p_prepare); residual: the packed 8-bit E8 table
  const uint32_t* tq_bad;
  const int32_t *te, *to, *tc;
  int64_t n_tiles, routes;
  int64_t E, N, K, G, kpg;  // kpg: K blocks per scale group
  float limit;
  void* out;
  int odt;
  int64_t ncb, total, per_xcd;  // column blocks, work items, items per XCD
  // the fused residual (HOT)
  const uint8_t *rc0, *rc1;  // residual codes [hot_rows][N][K / 8] (gate/up: gate, up)
  const void *rs0, *rs1;     // residual scales [hot_rows][N], one per row
  int rsdt;
  const int32_t* hot;        // residual row of each expert (-1: none)
  int64_t hot_rows;
  const uint32_t* t8;        // the packed 8-bit E8 table (uint32[256])
};

// RES: the nested tier's 8-bit E8 residual instead of E8P base codes (one code
// byte per codeword, one 8-byte lookup); the result is added to the fp32
// output (the base projection's). HOT: E8P base codes and, on the tiles of an
// expert with a residual row (hot[e] in [0, hot_rows)), that row's 8-bit E8
// residual codes, decoded from a second LDS image and multiplied by the same A
// operands into a second accumulator; base and residual are scaled and summed
// before the epilogue (the SwiGLU of gate/up), as the nested tier's serving
// step adds them (omlx_lattice.py:172-186). A hot tile runs as one pass per 32
// routes (its second m-tile's accumulators hold the residual); a hot row out of
// range other than -1 makes the tile's rows NaN. XT: the A rows' element type.
// NTW: 32-column n-tiles per wave (2: items of 512 columns; 1: of 256, for
// problems with too few items to spread over the CUs).
template <bool GATEUP, bool GROUPED, typename XT, bool RES = false, int NTW = 2, bool HOT = false>
__global__ __launch_bounds__(GQ_THREADS) void k_gemm_e8(GQArgs a) {
  static_assert(!(HOT && (RES || GROUPED)), "the fused residual takes E8P base codes and per-row scales");
  constexpr int D = 2;                         // K blocks in flight
  constexpr int NCOL = GQ_WAVES * 32 * NTW;    // output columns per work item
  constexpr int XV = sizeof(XT) == 4 ? 4 : 2;           // 16-byte A loads per thread and K block
  __shared__ uint4 tqs[TQR_BYTES / 16];
  __shared__ uint2 t8s[HOT ? T8R_BYTES / 8 : 1];  // HOT: the residual image
  __shared__ __attribute__((aligned(16))) uint8_t ash[2][GQ_M * GQ_ROW];
  __shared__ float s_ok[GQ_M];  // 1 / r of the row (NaN: no valid row)
  __shared__ int32_t s_orow[GQ_M];
  const char* img = (const char*)tqs;
  const char* img8 = (const char*)t8s;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c = lane & 31, h = lane >> 5;
  const Q8Keys lk = q8_keys(lane);
  const uint32_t tq_bad = GATEUP ? ((const __attribute__((address_space(4))) uint32_t*)a.tq_bad)[0] : 0u;
  {  // the LDS image(s): entry tid / 2, copies 8 (tid & 1) .. + 7
    const int e = tid >> 1;
    // residual row e: sixteen copies of the 8 bytes 2 (nibble d - 8) + 128, d = 0..7
    auto e8_row = [&](uint32_t p, char* base) {
      uint32_t b[2] = {0u, 0u};
#pragma unroll
      for (int d = 0; d < 8; ++d) b[d >> 2] |= ((uint32_t)(2 * ((int)((p >> (4 * d)) & 15u) - 8) + 128) & 0xffu) << (8 * (d & 3));
      uint2* row = (uint2*)(base + e * 128 + (tid & 1) * 64);
#pragma unroll
      for (int i = 0; i < 8; ++i) row[i] = make_uint2(b[0], b[1]);
    };
    if constexpr (RES) {
      e8_row(((const uint32_t*)a.tq)[e], (char*)tqs);
    } else {  // row e: sixteen copies of (T'[e], M[e]), T' = T ^ 0x80 per byte, natural dim order
      const uint2 t = gq_natural(((const uint2*)a.tq)[e]), m = gq_natural(((const uint2*)a.tq)[256 + e]);
      const uint4 v = make_uint4(t.x ^ 0x80808080u, t.y ^ 0x80808080u, m.x, m.y);
      uint4* row = tqs + e * 16 + (tid & 1) * 8;
#pragma unroll
      for (int i = 0; i < 8; ++i) row[i] = v;
      if constexpr (HOT) e8_row(a.t8[e], (char*)t8s);
    }
  }
  __syncthreads();

  const int64_t C = a.K >> 3;
  const int nkb = (int)(a.K / GQ_KB);
  const int xcd = blockIdx.x % GQ_XCDS;
  const int nb = gridDim.x / GQ_XCDS;
  // A staging: row sr, 8-element chunks sp and sp + 8 of its K block (the 8 threads of a row
  // write 128 consecutive LDS bytes per store: no bank conflicts)
  const int sr = tid >> 3, sp = tid & 7;
  const uint32_t sbytes = a.sdt == KEEP_F32 ? 4u : 2u;
  const uint32_t rbytes = a.rsdt == KEEP_F32 ? 4u : 2u;
  // B operand of k-step s of one n-tile from this lane's 8 codewords of the K
  // block, in two halves: the LDS image lookups (look), then the bytes -> fp16
  // (cvt), so that a k-step's lookups are issued two k-steps before its MFMAs.
  auto look = [&](const uint4& q, int s) -> uint4 {
    if constexpr (RES) {  // code bytes: codeword s is byte s of q.x / q.y
      const uint32_t w = s < 4 ? q.x : q.y;
      const uint32_t byte = (w >> (8 * (s & 3))) & 0xffu;
      const uint2 x = *(const uint2*)(img + byte * 128u + (uint32_t)(lane & 15) * 8u);
      return make_uint4(x.x, x.y, 0u, 0u);
    } else {
      const uint32_t w = s < 2 ? q.x : (s < 4 ? q.y : (s < 6 ? q.z : q.w));
      const bool hi = (s & 1) != 0;
      const uint32_t a1 = __builtin_amdgcn_perm(w, lk.base1, hi ? lk.s1hi : lk.s1lo);
      const uint32_t a2 = __builtin_amdgcn_perm(w, lk.base2, hi ? lk.s2hi : lk.s2lo);
      const uint2 x1 = *(const uint2*)(img + a1), x2 = *(const uint2*)(img + a2);
      return make_uint4(x1.x, x1.y, x2.x, x2.y);
    }
  };
  auto cvt = [&](const uint4& r) -> h8 { return gq_f16_of_bytes(make_uint2(r.x ^ r.z, r.y ^ r.w)); };
  // HOT: the residual codeword s of this lane's 8 code bytes -> its 8 bytes q + 128
  auto look_r = [&](const uint2& r, int s) -> uint2 {
    const uint32_t w = s < 4 ? r.x : r.y;
    const uint32_t byte = (w >> (8 * (s & 3))) & 0xffu;
    return *(const uint2*)(img8 + byte * 128u + (uint32_t)(lane & 15) * 8u);
  };

  // XCD-aware order: item w = column block x tiles + tile, each XCD running a
  // contiguous range of w, so the tiles of an expert at one column block (its
  // code rows) run side by side on one XCD and share its L2.
  for (int64_t j = blockIdx.x / GQ_XCDS; j < a.per_xcd; j += nb) {
    const int64_t w = xcd * a.per_xcd + j;
    if (w >= a.total) break;
    const int64_t cb = w / a.n_tiles, tile = w - cb * a.n_tiles;
    const int cnt_raw = a.tc[tile];
    const int64_t off = a.to[tile];
    const int cnt = min(cnt_raw, GQ_M);
    if (cnt_raw <= 0 || off < 0 || off + cnt > a.routes) continue;  // nothing can be written safely
    const int64_t e = a.te[tile];
    if (RES && e < 0) continue;  // routes off the residual tier (row -1): nothing to add
    bool bad = e < 0 || e >= a.E || cnt_raw > GQ_M;  // rows written as NaN
    int64_t hr = -1;  // HOT: the tile's residual row
    if constexpr (HOT) {
      if (!bad) {
        const int32_t r = a.hot[e];
        if (r >= 0 && r < a.hot_rows) hr = r;
        else if (r != -1) bad = true;
      }
    }
    const bool two = cnt > 32;

    // this lane's column of each n-tile: a code row and its scale row (HOT: and
    // its residual code row)
    int64_t n[NTW], crow[NTW], rrow[NTW];
    bool nv[NTW];
    const uint8_t* cp[NTW];
    const uint8_t* rp[NTW];
    const void* sbase[NTW];
    const void* rsbase[NTW];
#pragma unroll
    for (int jn = 0; jn < NTW; ++jn) {
      const uint16_t* cbase;
      const uint8_t* rbase;
      if constexpr (GATEUP) {
        n[jn] = cb * (NCOL / 2) + (wv * NTW + jn) * 16 + (c & 15);
        cbase = c < 16 ? a.c0 : a.c1;
        sbase[jn] = c < 16 ? a.s0 : a.s1;
        rbase = c < 16 ? a.rc0 : a.rc1;
        rsbase[jn] = c < 16 ? a.rs0 : a.rs1;
      } else {
        n[jn] = cb * NCOL + (wv * NTW + jn) * 32 + c;
        cbase = a.c0;
        sbase[jn] = a.s0;
        rbase = a.rc0;
        rsbase[jn] = a.rs0;
      }
      nv[jn] = n[jn] < a.N;
      crow[jn] = (bad || !nv[jn]) ? 0 : e * a.N + n[jn];
      // E8P: 16 bytes per K block (codewords 8 h ..); residual: 8 bytes (one byte per codeword)
      cp[jn] = RES ? (const uint8_t*)cbase + crow[jn] * C + 8 * h : (const uint8_t*)(cbase + crow[jn] * C + 8 * h);
      rrow[jn] = (hr < 0 || !nv[jn]) ? 0 : hr * a.N + n[jn];
      rp[jn] = HOT ? rbase + rrow[jn] * C + 8 * h : nullptr;
    }
    // A staging row of this thread
    int64_t xs = off + min(sr, cnt - 1);
    xs = a.lhs ? (int64_t)a.lhs[xs] : xs;
    if (xs < 0 || xs >= a.x_rows) xs = 0;
    const uint8_t* ap = (const uint8_t*)a.x + (xs * a.K + 8 * sp) * (int64_t)sizeof(XT);
    const float rsc = a.rs ? a.rs[xs].x : 1.f;  // this thread's row factor r
    // every wave has left the previous item's epilogue, which reads s_ok and
    // s_orow after the run loop's last barrier (block-uniform: every skip
    // above is taken by the whole block)
    __syncthreads();
    if (tid < GQ_M) {
      const int64_t pos = off + min(tid, cnt - 1);
      const int64_t xr = a.lhs ? (int64_t)a.lhs[pos] : pos;
      s_ok[tid] = (xr >= 0 && xr < a.x_rows) ? (a.rs ? a.rs[xr].y : 1.f) : __builtin_nanf("");
      s_orow[tid] = a.oidx ? a.oidx[pos] : (int32_t)pos;
    }

    struct Buf {
      uint4 q[NTW], ax[XV];  // codes of block u, A row elements of block u + 1
      uint2 r[NTW];          // HOT: residual codes of block u
    };
    auto issue = [&](int u, Buf& b, auto ht_c) {
      constexpr bool HT = decltype(ht_c)::value;
      const int kq = min(u, nkb - 1), ka = min(u + 1, nkb - 1);
#pragma unroll
      for (int jn = 0; jn < NTW; ++jn) {
        if constexpr (RES) {
          const uint2 v = ldg8_q(cp[jn] + kq * 16);
          b.q[jn] = make_uint4(v.x, v.y, 0u, 0u);
        } else {
          b.q[jn] = ldg16_q(cp[jn] + kq * 32);
        }
        if constexpr (HT) b.r[jn] = ldg8_q(rp[jn] + kq * 16);
      }
#pragma unroll
      for (int i = 0; i < XV; ++i) b.ax[i] = ldg16_q(ap + ((int64_t)ka * GQ_KB + 64 * (i / (XV / 2))) * sizeof(XT) +
                                                     16 * (i % (XV / 2)));
    };
    // 16 elements of the row (x r for bf16 / fp32) -> fp16 (round to nearest even), into the A buffer
    auto stage = [&](int buf, const uint4 (&ax)[XV]) {
      uint4 o[2];
      if constexpr (sizeof(XT) == 2 && !std::is_same<XT, bf16s>::value) {
        o[0] = ax[0];
        o[1] = ax[1];
      } else {
        uint32_t* ow = (uint32_t*)o;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          float f0, f1;
          if constexpr (sizeof(XT) == 4) {
            const uint32_t* xw = (const uint32_t*)ax;
            f0 = __uint_as_float(xw[2 * i]);
            f1 = __uint_as_float(xw[2 * i + 1]);
          } else {
            const uint32_t wd = ((const uint32_t*)ax)[i];
            f0 = __uint_as_float(wd << 16);
            f1 = __uint_as_float(wd & 0xffff0000u);
          }
          const h2v hv = {(_Float16)(f0 * rsc), (_Float16)(f1 * rsc)};
          ow[i] = __builtin_bit_cast(uint32_t, hv);
        }
      }
      uint8_t* d = &ash[buf][sr * GQ_ROW + 16 * sp];
      *(uint4*)d = o[0];
      *(uint4*)(d + 128) = o[1];
    };

    f32x16 acc[2][NTW];
    float accf[2][NTW][GROUPED ? 16 : 1];
    auto fold = [&](int g) {  // scale group g ends: add its partial sums
      if constexpr (GROUPED) {
#pragma unroll
        for (int jn = 0; jn < NTW; ++jn) {
          const int64_t si = crow[jn] * a.G + g;
          const float sc = nv[jn] && !bad ? scale_cvt(ldg4_q((const char*)sbase[jn] + ((si * sbytes) & ~(int64_t)3)),
                                                      a.sdt, (uint32_t)si)
                                          : 0.f;
#pragma unroll
          for (int mt = 0; mt < 2; ++mt) {
#pragma unroll
            for (int v = 0; v < 16; ++v) accf[mt][jn][v] = fmaf(acc[mt][jn][v], sc, accf[mt][jn][v]);
            acc[mt][jn] = f32x16{};
          }
        }
      }
    };
    // One pass over K. NT live m-tiles (from m-tile msel when NT = 1); HT: the
    // residual into acc[1] beside the base of m-tile msel into acc[0]. The
    // pass stages block 0's A rows and issues D blocks' loads, then unit u
    // stages the A rows of block u + 1, runs the MFMAs of block u k-step by
    // k-step and issues the loads of block u + D. During k-step s it looks up
    // the image for k-step s + 2 and converts the lookups of k-step s + 1
    // (issued one k-step earlier), so no lookup is waited on right after its
    // issue; the last two k-steps look up block u + 1's first two.
    auto pass = [&](auto nt_c, auto ht_c, int msel) {
      constexpr int NT = decltype(nt_c)::value;
      constexpr bool HT = decltype(ht_c)::value;
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int jn = 0; jn < NTW; ++jn) {
          acc[mt][jn] = f32x16{};
#pragma unroll
          for (int v = 0; v < (GROUPED ? 16 : 1); ++v) accf[mt][jn][v] = 0.f;
        }
      {
        uint4 ax0[XV];
#pragma unroll
        for (int i = 0; i < XV; ++i) ax0[i] = ldg16_q(ap + 64 * (i / (XV / 2)) * sizeof(XT) + 16 * (i % (XV / 2)));
        wait_vm_q<0>();
        stage(0, ax0);
      }
      Buf bb[D];
#pragma unroll
      for (int i = 0; i < D; ++i) issue(i, bb[i], ht_c);
      __syncthreads();  // A block 0, s_ok, s_orow; the previous pass's readers are done

      h8 Bc[NTW], Rc[NTW];
      uint4 Lc[NTW];
      uint2 Lr[NTW];
#pragma unroll
      for (int jn = 0; jn < NTW; ++jn) {
        Bc[jn] = cvt(look(bb[0].q[jn], 0));
        Lc[jn] = look(bb[0].q[jn], 1);
        if constexpr (HT) {
          Rc[jn] = gq_f16_of_bytes(look_r(bb[0].r[jn], 0));
          Lr[jn] = look_r(bb[0].r[jn], 1);
        }
      }
      auto unit = [&](int u, Buf& b, const Buf& bn) {
        stage((u + 1) & 1, b.ax);
        if (u < nkb) {
          const uint8_t* abase = &ash[u & 1][(c + 32 * msel) * GQ_ROW + 128 * h];
#pragma unroll
          for (int s = 0; s < 8; ++s) {
            h8 A[NT];
#pragma unroll
            for (int mt = 0; mt < NT; ++mt) A[mt] = *(const h8*)(abase + mt * 32 * GQ_ROW + 16 * s);
            uint4 Ln[NTW];
            uint2 Lrn[NTW];
            h8 Bn[NTW], Rn[NTW];
#pragma unroll
            for (int jn = 0; jn < NTW; ++jn) {
              Ln[jn] = s < 6 ? look(b.q[jn], s + 2) : look(bn.q[jn], s - 6);
              Bn[jn] = cvt(Lc[jn]);
              if constexpr (HT) {
                Lrn[jn] = s < 6 ? look_r(b.r[jn], s + 2) : look_r(bn.r[jn], s - 6);
                Rn[jn] = gq_f16_of_bytes(Lr[jn]);
              }
            }
#pragma unroll
            for (int jn = 0; jn < NTW; ++jn) {
#pragma unroll
              for (int mt = 0; mt < NT; ++mt) acc[mt][jn] = mfma32_f16(A[mt], Bc[jn], acc[mt][jn]);
              if constexpr (HT) acc[1][jn] = mfma32_f16(A[0], Rc[jn], acc[1][jn]);
            }
#pragma unroll
            for (int jn = 0; jn < NTW; ++jn) {
              Bc[jn] = Bn[jn];
              Lc[jn] = Ln[jn];
              if constexpr (HT) {
                Rc[jn] = Rn[jn];
                Lr[jn] = Lrn[jn];
              }
            }
          }
          if constexpr (GROUPED) {
            if ((u + 1) % a.kpg == 0) fold(u / (int)a.kpg);
          }
        }
        issue(u + D, b, ht_c);
        __syncthreads();
      };
      for (int u = 0; u < nkb; u += D) {  // every call unconditional: blocks past the end only reload
#pragma unroll
        for (int i = 0; i < D; ++i) unit(u + i, bb[i], bb[(i + 1) % D]);
      }
      wait_vm_q<0>();
    };

    // epilogue of a pass: D row m = 8 (v / 4) + 4 h + v % 4 of m-tile mt (HT:
    // of m-tile msel, base in acc[0] and residual in acc[1]), column c of n-tile jn
    auto emit = [&](auto ht_c, int msel) {
      constexpr bool HT = decltype(ht_c)::value;
#pragma unroll
      for (int jn = 0; jn < NTW; ++jn) {
        float sc = 0.25f, scr = 0.f;
        if constexpr (!GROUPED) {
          sc = nv[jn] && !bad ? 0.25f * scale_cvt(ldg4_q((const char*)sbase[jn] + ((crow[jn] * sbytes) & ~(int64_t)3)),
                                                  a.sdt, (uint32_t)crow[jn])
                              : 0.f;
        }
        if constexpr (HT) {
          scr = nv[jn] && !bad ? 0.25f * scale_cvt(ldg4_q((const char*)rsbase[jn] + ((rrow[jn] * rbytes) & ~(int64_t)3)),
                                                   a.rsdt, (uint32_t)rrow[jn])
                               : 0.f;
        }
#pragma unroll
        for (int mt = 0; mt < (HT ? 1 : 2); ++mt) {
#pragma unroll
          for (int v = 0; v < 16; ++v) {
            const int m = (HT ? msel : mt) * 32 + 8 * (v >> 2) + 4 * h + (v & 3);
            float val;
            if constexpr (HT) val = fmaf(acc[0][jn][v], sc, acc[1][jn][v] * scr) * s_ok[m];
            else val = (GROUPED ? accf[mt][jn][v] : acc[mt][jn][v]) * sc * s_ok[m];
            if (bad) val = __builtin_nanf("");
            if constexpr (GATEUP) {
              const float other = __shfl_xor(val, 16, 64);
              float hv = c < 16 ? silu_mul(val, other, a.limit) : silu_mul(other, val, a.limit);
              if (tq_bad) hv = __builtin_nanf("");
              const bool mine = (c < 16) == ((v & 1) == 0);
              if (mine && m < cnt && nv[jn])
                ((uint16_t*)a.out)[(off + m) * a.N + n[jn]] = from_float<bf16s>(hv).bits;
            } else {
              if (m < cnt && nv[jn]) {
                const int64_t o = (int64_t)s_orow[m] * a.N + n[jn];
                if constexpr (RES) ((float*)a.out)[o] += val;
                else if (a.odt == KEEP_F32) ((float*)a.out)[o] = val;
                else if (a.odt == KEEP_BF16) ((uint16_t*)a.out)[o] = from_float<bf16s>(val).bits;
                else ((_Float16*)a.out)[o] = (_Float16)val;
              }
            }
          }
        }
      }
    };

    using I1 = std::integral_constant<int, 1>;
    using I2 = std::integral_constant<int, 2>;
    using Cold = std::false_type;
    if (HOT && hr >= 0) {
      for (int ms = 0; ms < (two ? 2 : 1); ++ms) {
        pass(I1{}, std::integral_constant<bool, HOT>{}, ms);
        emit(std::integral_constant<bool, HOT>{}, ms);
      }
    } else {
      if (two) pass(I2{}, Cold{}, 0);
      else pass(I1{}, Cold{}, 0);
      emit(Cold{}, 0);
    }
  }
}

// ------------------------------------------------------------------ route combine

// out[t, :] = sum over j < k, in order, of w[t, j] * y[t k + j, :] (fp32
// multiply-adds: a NaN row stays NaN whatever its weight, as the reference's
// (y * scores[..., None]).sum(-2) keeps it). Four columns per thread.
__global__ __launch_bounds__(256) void k_route_combine(const float* y, const float* w, int64_t T, int k, int64_t H,
                                                       void* out, int odt) {
  const int64_t H4 = H >> 2;
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= T * H4) return;
  const int64_t t = i / H4, c = i - t * H4;
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int j = 0; j < k; ++j) {
    const float wt = w[t * k + j];
    const float4 v = ((const float4*)(y + (t * k + j) * H))[c];
    acc.x = fmaf(wt, v.x, acc.x);
    acc.y = fmaf(wt, v.y, acc.y);
    acc.z = fmaf(wt, v.z, acc.z);
    acc.w = fmaf(wt, v.w, acc.w);
  }
  const int64_t o = t * H + 4 * c;
  if (odt == KEEP_F32) {
    ((float4*)((float*)out + o))[0] = acc;
  } else if (odt == KEEP_BF16) {
    uint16_t* p = (uint16_t*)out + o;
    p[0] = from_float<bf16s>(acc.x).bits; p[1] = from_float<bf16s>(acc.y).bits;
    p[2] = from_float<bf16s>(acc.z).bits; p[3] = from_float<bf16s>(acc.w).bits;
  } else {
    _Float16* p = (_Float16*)out + o;
    p[0] = (_Float16)acc.x; p[1] = (_Float16)acc.y; p[2] = (_Float16)acc.z; p[3] = (_Float16)acc.w;
  }
}

// ------------------------------------------------------------------ host side

// Workspace: the row factors of bf16 / fp32 rows.
int64_t gq_ws_bytes(int64_t rows) { return (rows * (int64_t)sizeof(float2) + 255) / 256 * 256; }

const float2* gq_rowscale(const void* x, int x_dtype, int64_t rows, int64_t K, void* ws, hipStream_t s) {
  if (x_dtype == KEEP_F16) return nullptr;
  float2* rs = (float2*)ws;
  const dim3 grid((unsigned)((rows + 3) / 4));
  if (x_dtype == KEEP_BF16)
    hipLaunchKernelGGL((k_gq_rowscale<bf16s>), grid, dim3(256), 0, s, (const bf16s*)x, rows, (int)K, rs);
  else
    hipLaunchKernelGGL((k_gq_rowscale<float>), grid, dim3(256), 0, s, (const float*)x, rows, (int)K, rs);
  return rs;
}

template <bool GATEUP, bool RES, typename XT, int NTW, bool HOT>
void gq_launch_x(const GQArgs& a, dim3 grid, hipStream_t s) {
  if constexpr (HOT) hipLaunchKernelGGL((k_gemm_e8<GATEUP, false, XT, false, NTW, true>), grid, dim3(GQ_THREADS), 0, s, a);
  else if (a.G > 1) hipLaunchKernelGGL((k_gemm_e8<GATEUP, true, XT, RES, NTW>), grid, dim3(GQ_THREADS), 0, s, a);
  else hipLaunchKernelGGL((k_gemm_e8<GATEUP, false, XT, RES, NTW>), grid, dim3(GQ_THREADS), 0, s, a);
}

template <bool GATEUP, bool RES, int NTW, bool HOT = false>
void gq_launch_t(const GQArgs& a, dim3 grid, hipStream_t s) {
  if (a.xdt == KEEP_F16) gq_launch_x<GATEUP, RES, _Float16, NTW, HOT>(a, grid, s);
  else if (a.xdt == KEEP_BF16) gq_launch_x<GATEUP, RES, bf16s, NTW, HOT>(a, grid, s);
  else gq_launch_x<GATEUP, RES, float, NTW, HOT>(a, grid, s);
}

// hot: the fused residual (a.hot, a.rc0 / a.rc1, ... set; per-row scales)
void gq_launch(GQArgs& a, bool gateup, hipStream_t s, bool res = false, bool hot = false) {
  int dev = 0, cus = 256;
  if (hipGetDevice(&dev) == hipSuccess)
    (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  auto shape = [&](int64_t ncol) {
    const int64_t cols = gateup ? ncol / 2 : ncol;
    a.ncb = (a.N + cols - 1) / cols;
    a.total = a.ncb * a.n_tiles;
    a.per_xcd = (a.total + GQ_XCDS - 1) / GQ_XCDS;
  };
  shape(512);
  const bool wide = a.total >= 4 * (int64_t)cus;
  if (!wide) shape(256);
  const int64_t per = std::max<int64_t>(1, std::min<int64_t>(a.per_xcd, cus / GQ_XCDS));
  const dim3 grid((unsigned)(per * GQ_XCDS));
  if (wide) {
    if (hot) gateup ? gq_launch_t<true, false, 2, true>(a, grid, s) : gq_launch_t<false, false, 2, true>(a, grid, s);
    else if (res) gq_launch_t<false, true, 2>(a, grid, s);
    else if (gateup) gq_launch_t<true, false, 2>(a, grid, s);
    else gq_launch_t<false, false, 2>(a, grid, s);
  } else {
    if (hot) gateup ? gq_launch_t<true, false, 1, true>(a, grid, s) : gq_launch_t<false, false, 1, true>(a, grid, s);
    else if (res) gq_launch_t<false, true, 1>(a, grid, s);
    else if (gateup) gq_launch_t<true, false, 1>(a, grid, s);
    else gq_launch_t<false, false, 1>(a, grid, s);
  }
}

bool gq_shape_ok(int64_t K, int64_t group_size) {
  return K > 0 && K % GQ_KB == 0 && group_size > 0 && K % group_size == 0 && group_size % GQ_KB == 0 &&
         K <= (int64_t)1 << 20;
}

}  // namespace keep

using namespace keep;

// Workspace of the grouped GEMMs: one (r, 1 / r) pair per row of bf16 / fp32 input
// (fp16 input uses none).
extern "C" int64_t keep_vq_grouped_gemm_q8_workspace_bytes(int64_t x_rows, int64_t K) {
  if (!::keep::dims_ok({x_rows, K})) return -1;
  if (x_rows < 0 || K <= 0) return -1;
  return gq_ws_bytes(x_rows);
}

extern "C" int keep_vq_grouped_gemm_q8(const void* x, int x_dtype, int64_t x_rows, const int32_t* lhs,
                                       const int32_t* out_index, const void* codes, int code_bits, const void* scales,
                                       int scale_dtype, const void* prepared, const int32_t* tile_expert,
                                       const int32_t* tile_offset, const int32_t* tile_count, int64_t n_tiles,
                                       int64_t routes, int64_t num_experts, int64_t N, int64_t K, int64_t group_size,
                                       void* workspace, int64_t workspace_bytes, void* out, int out_dtype,
                                       void* stream) {
  KEEP_REQUIRE_DIMS(x_rows, n_tiles, routes, num_experts, N, K, group_size);
  KEEP_REQUIRE(x_dtype == KEEP_F16 || x_dtype == KEEP_BF16 || x_dtype == KEEP_F32, "bad activation dtype");
  KEEP_REQUIRE(dtype_ok(scale_dtype) && dtype_ok(out_dtype), "bad dtype enum");
  KEEP_REQUIRE(code_bits == 16 || code_bits == 8, "code_bits must be 16 (E8P) or 8 (residual E8)");
  KEEP_REQUIRE(code_bits == 16 || out_dtype == KEEP_F32, "the residual form adds into an fp32 output");
  KEEP_REQUIRE(gq_shape_ok(K, group_size),
               "grouped GEMM needs K and the scale group multiples of %d, the group dividing K (K=%lld, "
               "group_size=%lld)",
               GQ_KB, (long long)K, (long long)group_size);
  KEEP_REQUIRE(N > 0 && n_tiles >= 0 && routes >= 0 && num_experts > 0 && x_rows >= 0, "bad sizes");
  if (n_tiles == 0 || routes == 0) return KEEP_OK;
  KEEP_REQUIRE(x_rows > 0 && x && codes && scales && prepared && tile_expert && tile_offset && tile_count && out,
               "null pointer argument");
  KEEP_REQUIRE(aligned(x, 16) && aligned(codes, code_bits == 16 ? 16 : 8) && aligned(prepared, 16),
               "x and prepared must be 16-byte aligned, codes 16 (E8P) or 8 (residual) bytes");
  KEEP_REQUIRE(x_dtype == KEEP_F16 || (workspace && aligned(workspace, 16) && workspace_bytes >= gq_ws_bytes(x_rows)),
               "bf16 / fp32 input needs a 16-byte aligned workspace of %lld bytes, got %lld",
               (long long)gq_ws_bytes(x_rows), (long long)workspace_bytes);
  hipStream_t s = (hipStream_t)stream;
  GQArgs a{};
  a.x = x; a.xdt = x_dtype; a.x_rows = x_rows; a.lhs = lhs;
  a.rs = gq_rowscale(x, x_dtype, x_rows, K, workspace, s);
  a.oidx = out_index; a.c0 = a.c1 = (const uint16_t*)codes; a.s0 = a.s1 = scales; a.sdt = scale_dtype;
  if (code_bits == 8) {  // `prepared` is the packed 8-bit E8 table, uint32[256]
    a.tq = prepared;
    a.tq_bad = nullptr;
  } else {
    a.tq = (const char*)prepared + TQ_OFFSET;
    a.tq_bad = (const uint32_t*)((const char*)prepared + TQ_FLAG_OFFSET);
  }
  a.te = tile_expert; a.to = tile_offset; a.tc = tile_count; a.n_tiles = n_tiles; a.routes = routes;
  a.E = num_experts; a.N = N; a.K = K; a.G = K / group_size; a.kpg = group_size / GQ_KB; a.limit = 0.f;
  a.out = out; a.odt = out_dtype;
  gq_launch(a, false, s, code_bits == 8);
  return launch_status("keep_vq_grouped_gemm_q8");
}

extern "C" int keep_vq_grouped_swiglu_q8(const void* x, int x_dtype, int64_t x_rows, const int32_t* lhs,
                                         const uint16_t* gate_codes, const void* gate_scales,
                                         const uint16_t* up_codes, const void* up_scales, int scale_dtype,
                                         const void* prepared, const int32_t* tile_expert,
                                         const int32_t* tile_offset, const int32_t* tile_count, int64_t n_tiles,
                                         int64_t routes, int64_t num_experts, int64_t I, int64_t H,
                                         int64_t group_size, float swiglu_limit, void* workspace,
                                         int64_t workspace_bytes, void* h_out, void* stream) {
  KEEP_REQUIRE_DIMS(x_rows, n_tiles, routes, num_experts, I, H, group_size);
  KEEP_REQUIRE(x_dtype == KEEP_F16 || x_dtype == KEEP_BF16 || x_dtype == KEEP_F32, "bad activation dtype");
  KEEP_REQUIRE(dtype_ok(scale_dtype), "bad dtype enum");
  KEEP_REQUIRE(gq_shape_ok(H, group_size),
               "grouped GEMM needs H and the scale group multiples of %d, the group dividing H (H=%lld, "
               "group_size=%lld)",
               GQ_KB, (long long)H, (long long)group_size);
  KEEP_REQUIRE(I > 0 && n_tiles >= 0 && routes >= 0 && num_experts > 0 && x_rows >= 0, "bad sizes");
  if (n_tiles == 0 || routes == 0) return KEEP_OK;
  KEEP_REQUIRE(x_rows > 0 && x && gate_codes && gate_scales && up_codes && up_scales && prepared && tile_expert &&
                   tile_offset && tile_count && h_out,
               "null pointer argument");
  KEEP_REQUIRE(aligned(x, 16) && aligned(gate_codes, 16) && aligned(up_codes, 16) && aligned(prepared, 16),
               "x, codes and prepared must be 16-byte aligned");
  KEEP_REQUIRE(x_dtype == KEEP_F16 || (workspace && aligned(workspace, 16) && workspace_bytes >= gq_ws_bytes(x_rows)),
               "bf16 / fp32 input needs a 16-byte aligned workspace of %lld bytes, got %lld",
               (long long)gq_ws_bytes(x_rows), (long long)workspace_bytes);
  hipStream_t s = (hipStream_t)stream;
  GQArgs a{};
  a.x = x; a.xdt = x_dtype; a.x_rows = x_rows; a.lhs = lhs;
  a.rs = gq_rowscale(x, x_dtype, x_rows, H, workspace, s);
  a.oidx = nullptr; a.c0 = gate_codes; a.c1 = up_codes; a.s0 = gate_scales; a.s1 = up_scales;
  a.sdt = scale_dtype;
  a.tq = (const char*)prepared + TQ_OFFSET;
  a.tq_bad = (const uint32_t*)((const char*)prepared + TQ_FLAG_OFFSET);
  a.te = tile_expert; a.to = tile_offset; a.tc = tile_count; a.n_tiles = n_tiles; a.routes = routes;
  a.E = num_experts; a.N = I; a.K = H; a.G = H / group_size; a.kpg = group_size / GQ_KB; a.limit = swiglu_limit;
  a.out = h_out; a.odt = KEEP_BF16;
  gq_launch(a, true, s);
  return launch_status("keep_vq_grouped_swiglu_q8");
}

// The nested tier's checks and fields shared by the two fused-residual entry points.
static int gq_nested_args(GQArgs& a, const uint8_t* rc0, const void* rs0, const uint8_t* rc1, const void* rs1,
                          int res_scale_dtype, const int32_t* hot_row, int64_t hot_rows,
                          const uint32_t* res_table) {
  KEEP_REQUIRE(dtype_ok(res_scale_dtype), "bad dtype enum");
  KEEP_REQUIRE(hot_rows >= 0, "bad sizes");
  KEEP_REQUIRE(hot_row && res_table && rc0 && rs0 && rc1 && rs1, "null pointer argument");
  KEEP_REQUIRE(aligned(rc0, 8) && aligned(rc1, 8), "residual codes must be 8-byte aligned");
  a.rc0 = rc0; a.rc1 = rc1; a.rs0 = rs0; a.rs1 = rs1; a.rsdt = res_scale_dtype;
  a.hot = hot_row; a.hot_rows = hot_rows; a.t8 = res_table;
  return KEEP_OK;
}

extern "C" int keep_vq_grouped_swiglu_nested_q8(
    const void* x, int x_dtype, int64_t x_rows, const int32_t* lhs, const uint16_t* gate_codes,
    const void* gate_scales, const uint16_t* up_codes, const void* up_scales, int scale_dtype, const void* prepared,
    const uint8_t* gate_res_codes, const void* gate_res_scales, const uint8_t* up_res_codes,
    const void* up_res_scales, int res_scale_dtype, const int32_t* hot_row, int64_t hot_rows,
    const uint32_t* res_table, const int32_t* tile_expert, const int32_t* tile_offset, const int32_t* tile_count,
    int64_t n_tiles, int64_t routes, int64_t num_experts, int64_t I, int64_t H, float swiglu_limit,
    void* workspace, int64_t workspace_bytes, void* h_out, void* stream) {
  KEEP_REQUIRE_DIMS(x_rows, hot_rows, n_tiles, routes, num_experts, I, H);
  KEEP_REQUIRE(x_dtype == KEEP_F16 || x_dtype == KEEP_BF16 || x_dtype == KEEP_F32, "bad activation dtype");
  KEEP_REQUIRE(dtype_ok(scale_dtype), "bad dtype enum");
  KEEP_REQUIRE(gq_shape_ok(H, H), "grouped GEMM needs H a multiple of %d (H=%lld)", GQ_KB, (long long)H);
  KEEP_REQUIRE(I > 0 && n_tiles >= 0 && routes >= 0 && num_experts > 0 && x_rows >= 0, "bad sizes");
  if (n_tiles == 0 || routes == 0) return KEEP_OK;
  KEEP_REQUIRE(x_rows > 0 && x && gate_codes && gate_scales && up_codes && up_scales && prepared && tile_expert &&
                   tile_offset && tile_count && h_out,
               "null pointer argument");
  KEEP_REQUIRE(aligned(x, 16) && aligned(gate_codes, 16) && aligned(up_codes, 16) && aligned(prepared, 16),
               "x, codes and prepared must be 16-byte aligned");
  KEEP_REQUIRE(x_dtype == KEEP_F16 || (workspace && aligned(workspace, 16) && workspace_bytes >= gq_ws_bytes(x_rows)),
               "bf16 / fp32 input needs a 16-byte aligned workspace of %lld bytes, got %lld",
               (long long)gq_ws_bytes(x_rows), (long long)workspace_bytes);
  GQArgs a{};
  const int rc = gq_nested_args(a, gate_res_codes, gate_res_scales, up_res_codes, up_res_scales, res_scale_dtype,
                                hot_row, hot_rows, res_table);
  if (rc != KEEP_OK) return rc;
  hipStream_t s = (hipStream_t)stream;
  a.x = x; a.xdt = x_dtype; a.x_rows = x_rows; a.lhs = lhs;
  a.rs = gq_rowscale(x, x_dtype, x_rows, H, workspace, s);
  a.oidx = nullptr; a.c0 = gate_codes; a.c1 = up_codes; a.s0 = gate_scales; a.s1 = up_scales;
  a.sdt = scale_dtype;
  a.tq = (const char*)prepared + TQ_OFFSET;
  a.tq_bad = (const uint32_t*)((const char*)prepared + TQ_FLAG_OFFSET);
  a.te = tile_expert; a.to = tile_offset; a.tc = tile_count; a.n_tiles = n_tiles; a.routes = routes;
  a.E = num_experts; a.N = I; a.K = H; a.G = 1; a.kpg = H / GQ_KB; a.limit = swiglu_limit;
  a.out = h_out; a.odt = KEEP_BF16;
  gq_launch(a, true, s, false, true);
  return launch_status("keep_vq_grouped_swiglu_nested_q8");
}

extern "C" int keep_vq_grouped_gemm_nested_q8(
    const void* x, int x_dtype, int64_t x_rows, const int32_t* lhs, const int32_t* out_index, const uint16_t* codes,
    const void* scales, int scale_dtype, const void* prepared, const uint8_t* res_codes, const void* res_scales,
    int res_scale_dtype, const int32_t* hot_row, int64_t hot_rows, const uint32_t* res_table,
    const int32_t* tile_expert, const int32_t* tile_offset, const int32_t* tile_count, int64_t n_tiles,
    int64_t routes, int64_t num_experts, int64_t N, int64_t K, void* workspace, int64_t workspace_bytes, void* out,
    int out_dtype, void* stream) {
  KEEP_REQUIRE_DIMS(x_rows, hot_rows, n_tiles, routes, num_experts, N, K);
  KEEP_REQUIRE(x_dtype == KEEP_F16 || x_dtype == KEEP_BF16 || x_dtype == KEEP_F32, "bad activation dtype");
  KEEP_REQUIRE(dtype_ok(scale_dtype) && dtype_ok(out_dtype), "bad dtype enum");
  KEEP_REQUIRE(gq_shape_ok(K, K), "grouped GEMM needs K a multiple of %d (K=%lld)", GQ_KB, (long long)K);
  KEEP_REQUIRE(N > 0 && n_tiles >= 0 && routes >= 0 && num_experts > 0 && x_rows >= 0, "bad sizes");
  if (n_tiles == 0 || routes == 0) return KEEP_OK;
  KEEP_REQUIRE(x_rows > 0 && x && codes && scales && prepared && tile_expert && tile_offset && tile_count && out,
               "null pointer argument");
  KEEP_REQUIRE(aligned(x, 16) && aligned(codes, 16) && aligned(prepared, 16),
               "x, codes and prepared must be 16-byte aligned");
  KEEP_REQUIRE(x_dtype == KEEP_F16 || (workspace && aligned(workspace, 16) && workspace_bytes >= gq_ws_bytes(x_rows)),
               "bf16 / fp32 input needs a 16-byte aligned workspace of %lld bytes, got %lld",
               (long long)gq_ws_bytes(x_rows), (long long)workspace_bytes);
  GQArgs a{};
  const int rc = gq_nested_args(a, res_codes, res_scales, res_codes, res_scales, res_scale_dtype, hot_row, hot_rows,
                                res_table);
  if (rc != KEEP_OK) return rc;
  hipStream_t s = (hipStream_t)stream;
  a.x = x; a.xdt = x_dtype; a.x_rows = x_rows; a.lhs = lhs;
  a.rs = gq_rowscale(x, x_dtype, x_rows, K, workspace, s);
  a.oidx = out_index; a.c0 = a.c1 = codes; a.s0 = a.s1 = scales; a.sdt = scale_dtype;
  a.tq = (const char*)prepared + TQ_OFFSET;
  a.tq_bad = (const uint32_t*)((const char*)prepared + TQ_FLAG_OFFSET);
  a.te = tile_expert; a.to = tile_offset; a.tc = tile_count; a.n_tiles = n_tiles; a.routes = routes;
  a.E = num_experts; a.N = N; a.K = K; a.G = 1; a.kpg = K / GQ_KB; a.limit = 0.f;
  a.out = out; a.odt = out_dtype;
  gq_launch(a, false, s, false, true);
  return launch_status("keep_vq_grouped_gemm_nested_q8");
}

extern "C" int keep_route_combine(const float* y, const float* w, int64_t T, int64_t k, int64_t H, void* out,
                                  int out_dtype, void* stream) {
  KEEP_REQUIRE_DIMS(T, k, H);
  KEEP_REQUIRE(dtype_ok(out_dtype), "bad dtype enum");
  KEEP_REQUIRE(T >= 0 && k >= 1 && H >= 4 && H % 4 == 0, "need k >= 1 and H a multiple of 4");
  if (T == 0) return KEEP_OK;
  KEEP_REQUIRE(y && w && out, "null pointer argument");
  KEEP_REQUIRE(aligned(y, 16) && aligned(out, 16), "y and out must be 16-byte aligned");
  const int64_t n = T * (H / 4);
  hipLaunchKernelGGL(k_route_combine, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, (hipStream_t)stream, y, w, T,
                     (int)k, H, out, out_dtype);
  return launch_status("keep_route_combine");
}
