/*
 * CPU restatement of the routed E8P expert path -- TEST INFRASTRUCTURE ONLY
 * (the oracle's C form and the timed CPU baseline of bench.py; never linked
 * into keep_amd).
 *
 * Decode follows the reference decoder src/keep/vq/e8.py:203-234 bit by bit
 * (signs = c & 0xFF, idx = c >> 8, p = popcount(signs) & 1, eff = signs ^ p,
 * dim d reads nibble {0,4,1,5,2,6,3,7}[d], negated by bit of eff, +-1/4 by p).
 * The mat-vec decodes on the fly through a 65,536 x 8 float lookup table built
 * from that decoder (2 MiB, cache resident; no dense weight matrix), with
 * fp32 accumulation per scale group, OpenMP over (route, row). The MoE layer
 * is router outputs -> gate/up -> SwiGLU -> down -> weighted fp32 combine
 * (src/ramp/models/glm4_moe_adapter.py:367-372,
 * src/ramp/models/deepseek_v4_flash_adapter.py:962-967,1776-1784).
 *
 * Pins: oracle_e8p_decode is compared with the numpy oracle over all 65,536
 * codewords (tests/test_oracle_ops.py, test_c_oracle_decode_matches_numpy_oracle_everywhere), which is itself pinned by the
 * reference's golden vectors; the mat-vec and MoE layer against the float64
 * dense oracle.
 */
#include <math.h>
#include <omp.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

static const int kShuffle[8] = {0, 4, 1, 5, 2, 6, 3, 7};

void oracle_e8p_decode(const uint16_t* codes, int64_t n, const uint32_t* table, float* out) {
  for (int64_t i = 0; i < n; ++i) {
    uint32_t c = codes[i];
    uint32_t signs = c & 0xffu, idx = c >> 8;
    uint32_t p = 0;
    for (int b = 0; b < 8; ++b) p ^= (signs >> b) & 1u;
    uint32_t eff = signs ^ p;
    uint32_t word = table[idx];
    for (int d = 0; d < 8; ++d) {
      int s = kShuffle[d];
      float v = (float)((int)((word >> (4 * s)) & 15u) - 8) * 0.5f;
      if ((eff >> s) & 1u) v = -v;
      out[i * 8 + d] = v + (p ? -0.25f : 0.25f);
    }
  }
}

/* 65,536 x 8 decoded-value table for one codebook, cached across calls. */
static float* g_lut = NULL;
static uint32_t g_lut_table[256];

static const float* get_lut(const uint32_t* table) {
  if (g_lut && memcmp(g_lut_table, table, sizeof g_lut_table) == 0) return g_lut;
  if (!g_lut) g_lut = (float*)aligned_alloc(64, sizeof(float) * 65536 * 8);
  uint16_t* all = (uint16_t*)malloc(sizeof(uint16_t) * 65536);
  for (int i = 0; i < 65536; ++i) all[i] = (uint16_t)i;
  oracle_e8p_decode(all, 65536, table, g_lut);
  free(all);
  memcpy(g_lut_table, table, sizeof g_lut_table);
  return g_lut;
}

/* Dot of one code row (C codewords, G groups) with x (fp32). */
static inline float row_dot(const uint16_t* crow, const float* srow, int64_t C, int64_t cpg, const float* x,
                            const float* lut) {
  float total = 0.f;
  for (int64_t g0 = 0; g0 < C; g0 += cpg) {
    float acc = 0.f;
    for (int64_t c = g0; c < g0 + cpg; ++c) {
      const float* w = lut + (size_t)crow[c] * 8;
      const float* xv = x + c * 8;
      acc += w[0] * xv[0] + w[1] * xv[1] + w[2] * xv[2] + w[3] * xv[3] + w[4] * xv[4] + w[5] * xv[5] +
             w[6] * xv[6] + w[7] * xv[7];
    }
    total += acc * srow[g0 / cpg];
  }
  return total;
}

/* out[r, n] = W[rhs[r]][n, :] . x[lhs ? lhs[r] : r / x_div, :] */
void oracle_routed_matvec(const float* x, const uint16_t* codes, const float* scales, const uint32_t* table,
                          const int32_t* rhs, const int32_t* lhs, int64_t routes, int64_t x_div, int64_t N, int64_t K,
                          int64_t group_size, float* out, int threads) {
  const float* lut = get_lut(table);
  const int64_t C = K / 8, G = K / group_size, cpg = group_size / 8;
  if (threads > 0) omp_set_num_threads(threads);
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < routes * N; ++i) {
    const int64_t r = i / N, n = i % N;
    const int64_t e = rhs[r];
    const int64_t xr = lhs ? lhs[r] : r / x_div;
    out[i] = row_dot(codes + (e * N + n) * C, scales + (e * N + n) * G, C, cpg, x + xr * K, lut);
  }
}

/* 256 x 8 decoded values of a packed 8-bit E8 table (nibble d = dim d,
 * value (nibble - 8) / 2; src/keep/vq/e8.py:192-200). */
static void e8_lut(const uint32_t* table8, float* lut8) {
  for (int i = 0; i < 256; ++i)
    for (int d = 0; d < 8; ++d) lut8[i * 8 + d] = (float)((int)((table8[i] >> (4 * d)) & 15u) - 8) * 0.5f;
}

/* Dot of one 8-bit E8 code row (C codewords, G groups) with x (fp32). */
static inline float row_dot8(const uint8_t* crow, const float* srow, int64_t C, int64_t cpg, const float* x,
                             const float* lut8) {
  float total = 0.f;
  for (int64_t g0 = 0; g0 < C; g0 += cpg) {
    float acc = 0.f;
    for (int64_t c = g0; c < g0 + cpg; ++c) {
      const float* w = lut8 + (size_t)crow[c] * 8;
      const float* xv = x + c * 8;
      acc += w[0] * xv[0] + w[1] * xv[1] + w[2] * xv[2] + w[3] * xv[3] + w[4] * xv[4] + w[5] * xv[5] +
             w[6] * xv[6] + w[7] * xv[7];
    }
    total += acc * srow[g0 / cpg];
  }
  return total;
}

/* out[r, n] = dot(8-bit E8 code row (rhs[r], n), x row lhs[r] (or r / x_div)):
 * the nested tier's residual projection per route (rows rhs[r] of the residual
 * codes [nhot, N, K/8], scales [nhot, N, G]); routes with rhs[r] < 0 get 0. */
void oracle_routed_matvec8(const float* x, const uint8_t* codes, const float* scales, const uint32_t* table8,
                           const int32_t* rhs, const int32_t* lhs, int64_t routes, int64_t x_div, int64_t N, int64_t K,
                           int64_t group_size, float* out, int threads) {
  float lut8[256 * 8];
  e8_lut(table8, lut8);
  const int64_t C = K / 8, G = K / group_size, cpg = group_size / 8;
  if (threads > 0) omp_set_num_threads(threads);
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < routes * N; ++i) {
    const int64_t r = i / N, n = i % N;
    const int64_t e = rhs[r];
    const int64_t xr = lhs ? lhs[r] : r / x_div;
    out[i] = e < 0 ? 0.f : row_dot8(codes + (e * N + n) * C, scales + (e * N + n) * G, C, cpg, x + xr * K, lut8);
  }
}

/* Routed SwiGLU MoE for T tokens; x [T, H] fp32, scales fp32, out [T, H].
 * h_bf16 != 0 rounds the SwiGLU output to bf16 before the down projection.
 * With hot != NULL, the nested 3-bit tier: an expert e with hot[e] = r >= 0
 * adds the 8-bit E8 residual row r of each projection (codes uint8
 * [nhot, N, K/8], fp32 scales [nhot, N, K/rgroup]) to its E8P base before the
 * SwiGLU (gate, up) and before the weighted sum (down), as the nested mat-vec
 * src/ramp/kernels/e8p_nested_m1.metal:99-115 sums base and residual. */
void oracle_moe_decode_nested(const float* x, int64_t T, int64_t H, int64_t I, const int32_t* idx, const float* w,
                              int64_t k, const uint16_t* gc, const float* gs, const uint16_t* uc, const float* us,
                              const uint16_t* dc, const float* ds, int64_t group_h, int64_t group_i,
                              const uint32_t* table, float limit, int h_bf16, const int32_t* hot,
                              const uint8_t* rgc, const float* rgs, const uint8_t* ruc, const float* rus,
                              const uint8_t* rdc, const float* rds, int64_t rgroup_h, int64_t rgroup_i,
                              const uint32_t* table8, float* out, int threads) {
  const float* lut = get_lut(table);
  float lut8[256 * 8];
  if (hot) e8_lut(table8, lut8);
  float* h = (float*)malloc(sizeof(float) * T * k * I);
  const int64_t Ch = H / 8, Ci = I / 8, Gh = H / group_h, Gi = I / group_i;
  const int64_t RGh = hot ? H / rgroup_h : 1, RGi = hot ? I / rgroup_i : 1;
  if (threads > 0) omp_set_num_threads(threads);
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < T * k * I; ++i) {
    const int64_t route = i / I, n = i % I, t = route / k;
    const int64_t e = idx[route];
    float g = row_dot(gc + (e * I + n) * Ch, gs + (e * I + n) * Gh, Ch, group_h / 8, x + t * H, lut);
    float u = row_dot(uc + (e * I + n) * Ch, us + (e * I + n) * Gh, Ch, group_h / 8, x + t * H, lut);
    const int64_t r = hot ? hot[e] : -1;
    if (r >= 0) {
      g += row_dot8(rgc + (r * I + n) * Ch, rgs + (r * I + n) * RGh, Ch, rgroup_h / 8, x + t * H, lut8);
      u += row_dot8(ruc + (r * I + n) * Ch, rus + (r * I + n) * RGh, Ch, rgroup_h / 8, x + t * H, lut8);
    }
    if (limit > 0.f) {
      g = fminf(g, limit);
      u = fminf(fmaxf(u, -limit), limit);
    }
    float hv = g / (1.f + expf(-g)) * u;
    if (h_bf16) { /* round to bfloat16, nearest even (the reference stores h as bf16) */
      uint32_t b;
      memcpy(&b, &hv, 4);
      if ((b & 0x7fffffffu) <= 0x7f800000u) b = (b + 0x7fffu + ((b >> 16) & 1u)) & 0xffff0000u;
      memcpy(&hv, &b, 4);
    }
    h[i] = hv;
  }
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < T * H; ++i) {
    const int64_t t = i / H, n = i % H;
    float acc = 0.f;
    for (int64_t j = 0; j < k; ++j) {
      const int64_t route = t * k + j;
      const int64_t e = idx[route];
      float y = row_dot(dc + (e * H + n) * Ci, ds + (e * H + n) * Gi, Ci, group_i / 8, h + route * I, lut);
      const int64_t r = hot ? hot[e] : -1;
      if (r >= 0) y += row_dot8(rdc + (r * H + n) * Ci, rds + (r * H + n) * RGi, Ci, rgroup_i / 8, h + route * I, lut8);
      acc += w[route] * y;
    }
    out[i] = acc;
  }
  free(h);
}

void oracle_moe_decode(const float* x, int64_t T, int64_t H, int64_t I, const int32_t* idx, const float* w,
                       int64_t k, const uint16_t* gc, const float* gs, const uint16_t* uc, const float* us,
                       const uint16_t* dc, const float* ds, int64_t group_h, int64_t group_i,
                       const uint32_t* table, float limit, int h_bf16, float* out, int threads) {
  oracle_moe_decode_nested(x, T, H, I, idx, w, k, gc, gs, uc, us, dc, ds, group_h, group_i, table, limit, h_bf16,
                           NULL, NULL, NULL, NULL, NULL, NULL, NULL, 1, 1, NULL, out, threads);
}

/* Weighted nearest codeword by exhaustive scan (the definition the GPU
 * encoder keeps): for vector i (fp32 [8]) and weights w (NULL: 1; w_stride 0:
 * one shared [8]; 8: one [8] per vector) the grid index g minimising
 *   D = ((q0 + q1) + (q2 + q3)) + ((q4 + q5) + (q6 + q7)),  q_d = w_d * ((v_d - c_d)^2)
 * in double, ties to the lowest index (src/keep/quant/rtn.py:92-135, the
 * exhaustive reference of tests/test_e8p_diagonal_hessian.py:14-19). Each
 * statement rounds once: the file is built in ISO C mode (-std=c11), so no
 * multiply-add is contracted. */
void oracle_nearest(const float* v, int64_t n, const float* w, int64_t w_stride, const float* grid, int64_t G,
                    int64_t* out) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n; ++i) {
    double wd[8];
    for (int d = 0; d < 8; ++d) wd[d] = w ? (double)w[i * w_stride + d] : 1.0;
    double best = INFINITY;
    int64_t bi = 0;
    for (int64_t g = 0; g < G; ++g) {
      double q[8];
      for (int d = 0; d < 8; ++d) {
        const double df = (double)v[i * 8 + d] - (double)grid[g * 8 + d];
        const double sq = df * df;
        q[d] = wd[d] * sq;
      }
      const double a = q[0] + q[1], b = q[2] + q[3], c = q[4] + q[5], e = q[6] + q[7];
      const double ab = a + b, ce = c + e;
      const double D = ab + ce;
      if (D < best) {
        best = D;
        bi = g;
      }
    }
    out[i] = bi;
  }
}

int oracle_max_threads(void) { return omp_get_max_threads(); }
