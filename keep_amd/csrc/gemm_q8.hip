// Prefill grouped GEMM over expert-sorted routes on the int8 matrix cores
// (v_mfma_i32_32x32x32_i8), for tiles of up to 64 routes of one expert
// (the sorted-route prefill of src/ramp/ops/vq_switch.py:286-377 and
// glm4_moe_adapter.py:274-353: one route plan shared by gate, up and down).
//
// Operands.
//  * B = decoded weights x 4 (odd integers, |q| <= 15): T[idx] ^ M[signs]
//    from the 64 KiB LDS image, as the decode-layer kernels read it (see
//    q8_dev.h). A 32x32x32 MFMA takes 16 k of one column per lane (lane half
//    h = l / 32 holds k 16h .. 16h + 15); over a 128-wide K block, lane half
//    h loads codewords 8h .. 8h + 7 of its column (one 16-byte load) and at
//    k-step s feeds codewords 8h + 2s, 8h + 2s + 1 (q8_decode8's b[s]).
//  * A = activations as NTERM int8 terms under a per-row power of two s
//    (max |x| s in [32, 64)): x s = t0 + t1 / 128 (+ t2 / 128^2) + r. Three
//    terms for fp16 / fp32 rows (residual at most 2^-20 of the row's max, as
//    the decode layer's activations): gate/up outputs are rounded to bf16 in
//    h, and two terms (2^-13) flip that rounding often enough to cost ~1e-3
//    at the layer output. Three for bf16 rows (h of the down projection)
//    too: h is heavy tailed and two terms under the row's scale left 5.8e-3
//    of the output rms at single outputs of the 2048-token layer.
//    k_q8_rows writes the terms once per row ([row][term][K],
//    each codeword's 8 values in packed-nibble order), so the A bytes of lane
//    (m, h) at k-step s are row m's bytes 64h + 16s .. + 15 of the K block of
//    each term: the same k as B.
//  * D = (D0 + D1 / 128 + D2 / 128^2) / (4 s) x row scale, exact int32 sums per term.
//
// Block = 8 waves, one work item = (route tile, 256 output columns); wave w
// owns 32 columns and both 32-route m-tiles (the second is skipped when the
// tile holds <= 32 routes). The gate/up form pairs 16 gate rows with the same
// 16 up rows in a wave's 32 columns, so lanes l and l ^ 16 hold gate and up
// of one (route, row) and SwiGLU runs in the epilogue; h is written once, in
// bf16, at the route's sorted position.
//
// Pipeline. Persistent blocks (the LDS image is loaded once per block); a
// work item streams its K blocks with four blocks' code loads and A tiles
// in flight in registers (unrolled by four over four buffers, every load
// unconditional and clamped at the end), the A tile of the next block
// staged into a second LDS buffer while the current one feeds the MFMAs.
// Work items are spread XCD-aware: item w = column block x tiles + tile, and
// each XCD runs a contiguous range of w, so the tiles of an expert at one
// column block (sharing its code rows) run side by side on one XCD and hit
// its L2 (measured faster than keeping a tile's column blocks together).
#include <type_traits>

#include "common.h"
#include "moe_dev.h"
#include "q8_dev.h"

namespace keep {

constexpr int GQ_WAVES = 8;
constexpr int GQ_M = 64;                 // routes per tile (two 32-row m-tiles)
constexpr int GQ_KB = 128;               // k per K block
// LDS bytes per A row: the terms of one K block, padded so the rows of a
// 16-lane group start 4 banks apart (272 B) or 36 apart (400 B): no conflicts
template <int NTERM>
constexpr int gq_row() { return NTERM * GQ_KB + 16; }
constexpr int GQ_XCDS = 8;

typedef int i32x16 __attribute__((ext_vector_type(16)));

__device__ __forceinline__ i32x16 mfma32_i8(q8v4 a, q8v4 b, i32x16 c) {
  return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c, 0, 0, 0);
}

// ------------------------------------------------------------------ row terms

// One wave per row: s from max |x| (NaN anywhere in the row -> inv NaN), then
// the NTERM terms of each codeword's 8 values in packed-nibble order (dims
// 0, 2, 4, 6, 1, 3, 5, 7).
template <typename XT, int NTERM>
__global__ __launch_bounds__(256) void k_q8_rows(const XT* x, int64_t rows, int K, uint8_t* terms, float* inv) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int C = K >> 3;
  const XT* xr = x + row * K;
  auto load8 = [&](int c, float (&v)[8]) {
    if constexpr (sizeof(XT) == 4) {
      const float4 p = ((const float4*)(xr + 8 * c))[0], q = ((const float4*)(xr + 8 * c))[1];
      v[0] = p.x; v[1] = p.y; v[2] = p.z; v[3] = p.w; v[4] = q.x; v[5] = q.y; v[6] = q.z; v[7] = q.w;
    } else {
      const uint4 w = *(const uint4*)(xr + 8 * c);
      const uint32_t ww[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t lo = ww[i] & 0xffffu, hi = ww[i] >> 16;
        if constexpr (__is_same(XT, bf16s)) {
          v[2 * i] = __uint_as_float(lo << 16);
          v[2 * i + 1] = __uint_as_float(hi << 16);
        } else {
          v[2 * i] = (float)__builtin_bit_cast(_Float16, (uint16_t)lo);
          v[2 * i + 1] = (float)__builtin_bit_cast(_Float16, (uint16_t)hi);
        }
      }
    }
  };
  float mx = 0.f;
  bool nan = false;
  for (int c = lane; c < C; c += 64) {
    float v[8];
    load8(c, v);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      mx = fmaxf(mx, fabsf(v[i]));
      nan |= v[i] != v[i];
    }
  }
  mx = wave_max(mx);
  nan = __any(nan);
  float s, inv4s;
  q8_scale(mx, s, inv4s);
  if (nan) inv4s = __builtin_nanf("");
  uint8_t* t0 = terms + row * NTERM * K;
  for (int c = lane; c < C; c += 64) {
    float v[8];
    load8(c, v);
    const float p[4] = {v[0], v[2], v[4], v[6]}, q[4] = {v[1], v[3], v[5], v[7]};
    uint32_t lo[NTERM], hi[NTERM];
    q8_terms<NTERM>(p, s, lo);
    q8_terms<NTERM>(q, s, hi);
#pragma unroll
    for (int n = 0; n < NTERM; ++n) *(uint2*)(t0 + n * K + 8 * c) = make_uint2(lo[n], hi[n]);
  }
  if (lane == 0) inv[row] = inv4s;
}

// ------------------------------------------------------------------ grouped GEMM

struct GQArgs {
  const uint8_t* xt;   // [x_rows][2][K] int8 terms
  const float* xinv;   // [x_rows] 1 / (4 s)
  int64_t x_rows;
  const int32_t* lhs;   // sorted position -> A row (null: the position itself)
  const int32_t* oidx;  // sorted position -> output row (null: the position itself)
  const uint16_t *c0, *c1;  // codes [E][N][K / 8] (gate/up: gate, up)
  const void *s0, *s1;      // scales [E][N][G]
  int sdt;
  const uint4* tq;
  const uint32_t* tq_bad;
  const int32_t *te, *to, *tc;
  int64_t n_tiles, routes;
  int64_t E, N, K, G, kpg;  // kpg: K blocks per scale group
  float limit;
  void* out;
  int odt;
  int64_t ncb, total, per_xcd;  // column blocks, work items, items per XCD
};

// RES: the nested tier's 8-bit E8 residual instead of E8P base codes (t8_entry
// and t8_decode2 in q8_dev.h); the block builds the 32 KiB residual image from
// the packed table and the result is added to the fp32 output (the base
// projection's).
template <bool GATEUP, bool GROUPED, int NTERM, bool RES = false>
__global__ __launch_bounds__(512) void k_gemm_q8(GQArgs a) {
  constexpr int D = NTERM == 3 ? 3 : 4;  // K blocks in flight
  constexpr int ROW = gq_row<NTERM>();
  __shared__ uint4 tqs[TQR_BYTES / 16];
  __shared__ __attribute__((aligned(16))) uint8_t ash[2][GQ_M * ROW];
  __shared__ float s_inv[GQ_M];
  __shared__ int32_t s_orow[GQ_M];
  const char* tq = (const char*)tqs;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c = lane & 31, h = lane >> 5;
  const Q8Keys lk = q8_keys(lane);
  const uint32_t tq_bad = GATEUP ? ((const __attribute__((address_space(4))) uint32_t*)a.tq_bad)[0] : 0u;
  if constexpr (RES) {
    const uint2 v = t8_entry(((const uint32_t*)a.tq)[tid >> 1]);  // entry tid / 2, copies 8 (tid & 1) .. + 7
    uint2* row = (uint2*)((char*)tqs + (tid >> 1) * 128 + (tid & 1) * 64);
#pragma unroll
    for (int i = 0; i < 8; ++i) row[i] = v;
  } else {
#pragma unroll
    for (int u = 0; u < 8; ++u) dma16_q(a.tq + (wv * 8 + u) * 64 + lane, tqs + (wv * 8 + u) * 64);
  }
  wait_vm_q<0>();
  __syncthreads();

  const int64_t C = a.K >> 3;
  const int nkb = (int)(a.K / GQ_KB);
  const int xcd = blockIdx.x % GQ_XCDS;
  const int nb = gridDim.x / GQ_XCDS;
  const int sr = tid >> 3, sp = tid & 7;  // A staging: row sr, 16-byte chunk sp of each term
  // B operands of k-step s from a code word: E8P dword (two codewords) or two residual bytes
  auto decode = [&](uint32_t w) -> q8v4 {
    if constexpr (RES) {
      return t8_decode2(tq, (uint32_t)lane, w);
    } else {
      return q8_decode2(tq, lk, w);
    }
  };
  auto words = [&](const uint4& q, uint32_t (&w)[4]) {
    if constexpr (RES) {
      w[0] = q.x & 0xffffu; w[1] = q.x >> 16; w[2] = q.y & 0xffffu; w[3] = q.y >> 16;
    } else {
      w[0] = q.x; w[1] = q.y; w[2] = q.z; w[3] = q.w;
    }
  };
  const uint32_t sbytes = a.sdt == KEEP_F32 ? 4u : 2u;

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
    const bool bad = e < 0 || e >= a.E || cnt_raw > GQ_M;  // rows written as NaN
    const bool two = cnt > 32;

    // this lane's column: a code row and its scale row
    int64_t n;
    const uint16_t* cbase;
    const void* sbase;
    if constexpr (GATEUP) {
      n = cb * 128 + wv * 16 + (c & 15);
      cbase = c < 16 ? a.c0 : a.c1;
      sbase = c < 16 ? a.s0 : a.s1;
    } else {
      n = cb * 256 + wv * 32 + c;
      cbase = a.c0;
      sbase = a.s0;
    }
    const bool nv = n < a.N;
    const int64_t crow = (bad || !nv) ? 0 : e * a.N + n;
    const uint16_t* cp = cbase + crow * C + 8 * h;  // E8P: 16 bytes per K block
    const uint8_t* cp8 = (const uint8_t*)cbase + crow * C + 8 * h;  // residual: 8 bytes per K block
    // A staging row of this thread
    int64_t xs = off + min(sr, cnt - 1);
    xs = a.lhs ? (int64_t)a.lhs[xs] : xs;
    if (xs < 0 || xs >= a.x_rows) xs = 0;
    const uint8_t* ap = a.xt + xs * NTERM * a.K + 16 * sp;
    // every wave has left the previous item's epilogue, which reads s_inv and
    // s_orow after the run loop's last barrier (block-uniform: every skip
    // above is taken by the whole block)
    __syncthreads();
    if (tid < GQ_M) {
      const int64_t pos = off + min(tid, cnt - 1);
      const int64_t xr = a.lhs ? (int64_t)a.lhs[pos] : pos;
      s_inv[tid] = (xr >= 0 && xr < a.x_rows) ? a.xinv[xr] : __builtin_nanf("");
      s_orow[tid] = a.oidx ? a.oidx[pos] : (int32_t)pos;
    }

    struct Buf {
      uint4 q, at[NTERM];  // codes of block u, A terms of block u + 1
    };
    auto issue = [&](int u, Buf& b) {
      const int kq = min(u, nkb - 1), ka = min(u + 1, nkb - 1);
      if constexpr (RES) {
        const uint2 v = ldg8_q(cp8 + kq * 16);
        b.q = make_uint4(v.x, v.y, 0u, 0u);
      } else {
        b.q = ldg16_q(cp + kq * 16);
      }
#pragma unroll
      for (int t = 0; t < NTERM; ++t) b.at[t] = ldg16_q(ap + t * a.K + ka * GQ_KB);
    };
    auto stage = [&](int buf, const uint4 (&at)[NTERM]) {
      uint8_t* d = &ash[buf][sr * ROW + 16 * sp];
#pragma unroll
      for (int t = 0; t < NTERM; ++t) *(uint4*)(d + t * GQ_KB) = at[t];
    };
    {
      uint4 at0[NTERM];
#pragma unroll
      for (int t = 0; t < NTERM; ++t) at0[t] = ldg16_q(ap + t * a.K);
      wait_vm_q<0>();
      stage(0, at0);
    }
    Buf bb[D];
#pragma unroll
    for (int i = 0; i < D; ++i) issue(i, bb[i]);
    __syncthreads();  // A block 0, s_inv, s_orow; the previous item's readers are done

    i32x16 acc[2][NTERM];
    float accf[2][16];
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
#pragma unroll
      for (int t = 0; t < NTERM; ++t) acc[mt][t] = i32x16{};
#pragma unroll
      for (int v = 0; v < 16; ++v) accf[mt][v] = 0.f;
    }
    auto dot = [&](int mt, int v) {  // the K block sums of D element v, in units of 1 / (4 s)
      float d = (float)acc[mt][0][v] + (float)acc[mt][1][v] * 0.0078125f;
      if constexpr (NTERM == 3) d += (float)acc[mt][2][v] * 0.00006103515625f;
      return d;
    };
    auto fold = [&](int g) {  // scale group g ends: add its partial sums
      const float sc = nv && !bad ? scale_cvt(ldg4_q((const char*)sbase + (((crow * a.G + g) * sbytes) & ~(int64_t)3)),
                                              a.sdt, (uint32_t)(crow * a.G + g))
                                  : 0.f;
#pragma unroll
      for (int mt = 0; mt < 2; ++mt) {
#pragma unroll
        for (int v = 0; v < 16; ++v) accf[mt][v] += dot(mt, v) * sc;
#pragma unroll
        for (int t = 0; t < NTERM; ++t) acc[mt][t] = i32x16{};
      }
    };
    // NT live m-tiles. Unit u multiplies with the B operands of block u
    // (decoded during unit u - 1) while it decodes block u + 1 one dword per
    // k-step, stages the A terms of block u + 1 and issues the loads of
    // block u + D: the matrix cores run under the decode and the staging.
    q8v4 Bx[2][4];
    {
      uint32_t w4[4];
      words(bb[0].q, w4);
#pragma unroll
      for (int i = 0; i < 4; ++i) Bx[0][i] = decode(w4[i]);
    }
    auto run = [&](auto nt_c) {
      constexpr int NT = decltype(nt_c)::value;
      auto unit = [&](int u, Buf& b, const Buf& bn, const q8v4 (&Bc)[4], q8v4 (&Bn)[4]) {
        stage((u + 1) & 1, b.at);
        uint32_t wn[4];
        words(bn.q, wn);
        if (u < nkb) {
          const uint8_t* abase = &ash[u & 1][c * ROW + 64 * h];
#pragma unroll
          for (int s = 0; s < 4; ++s) {
            q8v4 A[NT][NTERM];
#pragma unroll
            for (int mt = 0; mt < NT; ++mt)
#pragma unroll
              for (int t = 0; t < NTERM; ++t) A[mt][t] = *(const q8v4*)(abase + mt * 32 * ROW + t * GQ_KB + 16 * s);
#pragma unroll
            for (int mt = 0; mt < NT; ++mt)
#pragma unroll
              for (int t = 0; t < NTERM; ++t) acc[mt][t] = mfma32_i8(A[mt][t], Bc[s], acc[mt][t]);
            Bn[s] = decode(wn[s]);
          }
          if constexpr (GROUPED) {
            if ((u + 1) % a.kpg == 0) fold(u / (int)a.kpg);
          }
        }
        issue(u + D, b);
        __syncthreads();
      };
      constexpr int UN = D % 2 == 0 ? D : 2 * D;  // a multiple of D (buffers) and of 2 (B operands)
      for (int u = 0; u < nkb; u += UN) {  // every call unconditional: blocks past the end only reload
#pragma unroll
        for (int i = 0; i < UN; ++i) unit(u + i, bb[i % D], bb[(i + 1) % D], Bx[i & 1], Bx[(i + 1) & 1]);
      }
    };
    if (two) run(std::integral_constant<int, 2>{});
    else run(std::integral_constant<int, 1>{});
    wait_vm_q<0>();

    // epilogue: D row m = 8 (v / 4) + 4 h + v % 4 of m-tile mt, column c
    float sc = 1.f;
    if constexpr (!GROUPED) {
      sc = nv && !bad ? scale_cvt(ldg4_q((const char*)sbase + ((crow * sbytes) & ~(int64_t)3)), a.sdt, (uint32_t)crow)
                      : 0.f;
    }
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int m = mt * 32 + 8 * (v >> 2) + 4 * h + (v & 3);
        float val;
        if constexpr (GROUPED) val = accf[mt][v] * s_inv[m];
        else val = dot(mt, v) * s_inv[m] * sc;
        if (bad) val = __builtin_nanf("");
        if constexpr (GATEUP) {
          const float other = __shfl_xor(val, 16, 64);
          float hv = c < 16 ? silu_mul(val, other, a.limit) : silu_mul(other, val, a.limit);
          if (tq_bad) hv = __builtin_nanf("");
          const bool mine = (c < 16) == ((v & 1) == 0);
          if (mine && m < cnt && nv)
            ((uint16_t*)a.out)[(off + m) * a.N + n] = from_float<bf16s>(hv).bits;
        } else {
          if (m < cnt && nv) {
            const int64_t o = (int64_t)s_orow[m] * a.N + n;
            if constexpr (RES) ((float*)a.out)[o] += val;
            else if (a.odt == KEEP_F32) ((float*)a.out)[o] = val;
            else if (a.odt == KEEP_BF16) ((uint16_t*)a.out)[o] = from_float<bf16s>(val).bits;
            else ((_Float16*)a.out)[o] = (_Float16)val;
          }
        }
      }
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

// Three terms for every row dtype. Two terms for bf16 rows (h of the down
// projection) leave a residual of 2^-13 of the row's maximum; h is heavy
// tailed (a row's maximum is ~12x its rms at config 4), and that residual
// measured 5.8e-3 of the output rms at single outputs of a 2048-token layer,
// where three terms leave 2^-20.
int gq_nterm(int) { return 3; }
int64_t gq_ws_terms(int64_t rows, int64_t K) { return (rows * 3 * K + 255) / 256 * 256; }
int64_t gq_ws_bytes(int64_t rows, int64_t K) { return gq_ws_terms(rows, K) + (rows * 4 + 255) / 256 * 256; }

void gq_rows(const void* x, int x_dtype, int64_t rows, int64_t K, uint8_t* ws, hipStream_t s) {
  const dim3 grid((unsigned)((rows + 3) / 4));
  uint8_t* terms = ws;
  float* inv = (float*)(ws + gq_ws_terms(rows, K));
  if (x_dtype == KEEP_F16)
    hipLaunchKernelGGL((k_q8_rows<_Float16, 3>), grid, dim3(256), 0, s, (const _Float16*)x, rows, (int)K, terms, inv);
  else if (x_dtype == KEEP_BF16)
    hipLaunchKernelGGL((k_q8_rows<bf16s, 3>), grid, dim3(256), 0, s, (const bf16s*)x, rows, (int)K, terms, inv);
  else
    hipLaunchKernelGGL((k_q8_rows<float, 3>), grid, dim3(256), 0, s, (const float*)x, rows, (int)K, terms, inv);
}

template <bool GATEUP, int NTERM>
void gq_launch_t(const GQArgs& a, dim3 grid, hipStream_t s) {
  if (a.G > 1) hipLaunchKernelGGL((k_gemm_q8<GATEUP, true, NTERM>), grid, dim3(512), 0, s, a);
  else hipLaunchKernelGGL((k_gemm_q8<GATEUP, false, NTERM>), grid, dim3(512), 0, s, a);
}

template <int NTERM>
void gq_launch_res(const GQArgs& a, dim3 grid, hipStream_t s) {
  if (a.G > 1) hipLaunchKernelGGL((k_gemm_q8<false, true, NTERM, true>), grid, dim3(512), 0, s, a);
  else hipLaunchKernelGGL((k_gemm_q8<false, false, NTERM, true>), grid, dim3(512), 0, s, a);
}

void gq_launch(GQArgs& a, bool gateup, int nterm, hipStream_t s, bool res = false) {
  a.ncb = gateup ? (a.N + 127) / 128 : (a.N + 255) / 256;
  a.total = a.ncb * a.n_tiles;
  a.per_xcd = (a.total + GQ_XCDS - 1) / GQ_XCDS;
  int dev = 0, cus = 256;
  if (hipGetDevice(&dev) == hipSuccess) hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  const int64_t per = std::max<int64_t>(1, std::min<int64_t>(a.per_xcd, cus / GQ_XCDS));
  const dim3 grid((unsigned)(per * GQ_XCDS));
  (void)nterm;  // always 3 (gq_nterm)
  if (res) gq_launch_res<3>(a, grid, s);
  else if (gateup) gq_launch_t<true, 3>(a, grid, s);
  else gq_launch_t<false, 3>(a, grid, s);
}

bool gq_shape_ok(int64_t K, int64_t group_size) {
  return K > 0 && K % GQ_KB == 0 && group_size > 0 && K % group_size == 0 && group_size % GQ_KB == 0 &&
         K <= (int64_t)1 << 20;
}

}  // namespace keep

using namespace keep;

extern "C" int64_t keep_vq_grouped_gemm_q8_workspace_bytes(int64_t x_rows, int64_t K) {
  if (x_rows < 0 || K <= 0) return -1;
  return gq_ws_bytes(x_rows, K);
}

extern "C" int keep_vq_grouped_gemm_q8(const void* x, int x_dtype, int64_t x_rows, const int32_t* lhs,
                                       const int32_t* out_index, const void* codes, int code_bits, const void* scales,
                                       int scale_dtype, const void* prepared, const int32_t* tile_expert,
                                       const int32_t* tile_offset, const int32_t* tile_count, int64_t n_tiles,
                                       int64_t routes, int64_t num_experts, int64_t N, int64_t K, int64_t group_size,
                                       void* workspace, int64_t workspace_bytes, void* out, int out_dtype,
                                       void* stream) {
  KEEP_REQUIRE(x_dtype == KEEP_F16 || x_dtype == KEEP_BF16 || x_dtype == KEEP_F32, "bad activation dtype");
  KEEP_REQUIRE(dtype_ok(scale_dtype) && dtype_ok(out_dtype), "bad dtype enum");
  KEEP_REQUIRE(code_bits == 16 || code_bits == 8, "code_bits must be 16 (E8P) or 8 (residual E8)");
  KEEP_REQUIRE(code_bits == 16 || out_dtype == KEEP_F32, "the residual form adds into an fp32 output");
  KEEP_REQUIRE(gq_shape_ok(K, group_size),
               "int8 grouped GEMM needs K and the scale group multiples of %d, the group dividing K (K=%lld, "
               "group_size=%lld)",
               GQ_KB, (long long)K, (long long)group_size);
  KEEP_REQUIRE(N > 0 && n_tiles >= 0 && routes >= 0 && num_experts > 0 && x_rows >= 0, "bad sizes");
  if (n_tiles == 0 || routes == 0) return KEEP_OK;
  KEEP_REQUIRE(x_rows > 0 && x && codes && scales && prepared && tile_expert && tile_offset && tile_count && out &&
                   workspace,
               "null pointer argument");
  KEEP_REQUIRE(workspace_bytes >= gq_ws_bytes(x_rows, K), "workspace needs %lld bytes, got %lld",
               (long long)gq_ws_bytes(x_rows, K), (long long)workspace_bytes);
  KEEP_REQUIRE(aligned(x, 16) && aligned(codes, code_bits == 16 ? 16 : 8) && aligned(prepared, 16) &&
                   aligned(workspace, 256),
               "x and prepared must be 16-byte aligned, codes 16 (E8P) or 8 (residual) bytes, the workspace 256");
  hipStream_t s = (hipStream_t)stream;
  uint8_t* ws = (uint8_t*)workspace;
  gq_rows(x, x_dtype, x_rows, K, ws, s);
  GQArgs a{};
  a.xt = ws; a.xinv = (const float*)(ws + gq_ws_terms(x_rows, K)); a.x_rows = x_rows; a.lhs = lhs;
  a.oidx = out_index; a.c0 = a.c1 = (const uint16_t*)codes; a.s0 = a.s1 = scales; a.sdt = scale_dtype;
  if (code_bits == 8) {  // `prepared` is the packed 8-bit E8 table, uint32[256]
    a.tq = (const uint4*)prepared;
    a.tq_bad = nullptr;
  } else {
    a.tq = (const uint4*)((const char*)prepared + TQR_OFFSET);
    a.tq_bad = (const uint32_t*)((const char*)prepared + TQ_FLAG_OFFSET);
  }
  a.te = tile_expert; a.to = tile_offset; a.tc = tile_count; a.n_tiles = n_tiles; a.routes = routes;
  a.E = num_experts; a.N = N; a.K = K; a.G = K / group_size; a.kpg = group_size / GQ_KB; a.limit = 0.f;
  a.out = out; a.odt = out_dtype;
  gq_launch(a, false, gq_nterm(x_dtype), s, code_bits == 8);
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
  KEEP_REQUIRE(x_dtype == KEEP_F16 || x_dtype == KEEP_BF16 || x_dtype == KEEP_F32, "bad activation dtype");
  KEEP_REQUIRE(dtype_ok(scale_dtype), "bad dtype enum");
  KEEP_REQUIRE(gq_shape_ok(H, group_size),
               "int8 grouped GEMM needs H and the scale group multiples of %d, the group dividing H (H=%lld, "
               "group_size=%lld)",
               GQ_KB, (long long)H, (long long)group_size);
  KEEP_REQUIRE(I > 0 && n_tiles >= 0 && routes >= 0 && num_experts > 0 && x_rows >= 0, "bad sizes");
  if (n_tiles == 0 || routes == 0) return KEEP_OK;
  KEEP_REQUIRE(x_rows > 0 && x && gate_codes && gate_scales && up_codes && up_scales && prepared && tile_expert &&
                   tile_offset && tile_count && h_out && workspace,
               "null pointer argument");
  KEEP_REQUIRE(workspace_bytes >= gq_ws_bytes(x_rows, H), "workspace needs %lld bytes, got %lld",
               (long long)gq_ws_bytes(x_rows, H), (long long)workspace_bytes);
  KEEP_REQUIRE(aligned(x, 16) && aligned(gate_codes, 16) && aligned(up_codes, 16) && aligned(prepared, 16) &&
                   aligned(workspace, 256),
               "x, codes and prepared must be 16-byte aligned, the workspace 256-byte aligned");
  hipStream_t s = (hipStream_t)stream;
  uint8_t* ws = (uint8_t*)workspace;
  gq_rows(x, x_dtype, x_rows, H, ws, s);
  GQArgs a{};
  a.xt = ws; a.xinv = (const float*)(ws + gq_ws_terms(x_rows, H)); a.x_rows = x_rows; a.lhs = lhs;
  a.oidx = nullptr; a.c0 = gate_codes; a.c1 = up_codes; a.s0 = gate_scales; a.s1 = up_scales;
  a.sdt = scale_dtype;
  a.tq = (const uint4*)((const char*)prepared + TQR_OFFSET);
  a.tq_bad = (const uint32_t*)((const char*)prepared + TQ_FLAG_OFFSET);
  a.te = tile_expert; a.to = tile_offset; a.tc = tile_count; a.n_tiles = n_tiles; a.routes = routes;
  a.E = num_experts; a.N = I; a.K = H; a.G = H / group_size; a.kpg = group_size / GQ_KB; a.limit = swiglu_limit;
  a.out = h_out; a.odt = KEEP_BF16;
  gq_launch(a, true, gq_nterm(x_dtype), s);
  return launch_status("keep_vq_grouped_swiglu_q8");
}

extern "C" int keep_route_combine(const float* y, const float* w, int64_t T, int64_t k, int64_t H, void* out,
                                  int out_dtype, void* stream) {
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
