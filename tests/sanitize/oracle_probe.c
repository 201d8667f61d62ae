/* The C oracle (oracle/cpu_ref.c) under AddressSanitizer and
 * UndefinedBehaviorSanitizer: every exported function on small exact-size
 * buffers (empty inputs, absent routes of the nested tier, shared and
 * per-vector weights, limits, bf16 rounding of h including non-finite
 * values). Any out-of-bounds access or undefined behaviour aborts. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>

void oracle_e8p_decode(const uint16_t* codes, int64_t n, const uint32_t* table, float* out);
void oracle_routed_matvec(const float* x, const uint16_t* codes, const float* scales, const uint32_t* table,
                          const int32_t* rhs, const int32_t* lhs, int64_t routes, int64_t x_div, int64_t N, int64_t K,
                          int64_t group_size, float* out, int threads);
void oracle_routed_matvec8(const float* x, const uint8_t* codes, const float* scales, const uint32_t* table8,
                           const int32_t* rhs, const int32_t* lhs, int64_t routes, int64_t x_div, int64_t N, int64_t K,
                           int64_t group_size, float* out, int threads);
void oracle_moe_decode_nested(const float* x, int64_t T, int64_t H, int64_t I, const int32_t* idx, const float* w,
                              int64_t k, const uint16_t* gc, const float* gs, const uint16_t* uc, const float* us,
                              const uint16_t* dc, const float* ds, int64_t group_h, int64_t group_i,
                              const uint32_t* table, float limit, int h_bf16, const int32_t* hot,
                              const uint8_t* rgc, const float* rgs, const uint8_t* ruc, const float* rus,
                              const uint8_t* rdc, const float* rds, int64_t rgroup_h, int64_t rgroup_i,
                              const uint32_t* table8, float* out, int threads);
void oracle_moe_decode(const float* x, int64_t T, int64_t H, int64_t I, const int32_t* idx, const float* w,
                       int64_t k, const uint16_t* gc, const float* gs, const uint16_t* uc, const float* us,
                       const uint16_t* dc, const float* ds, int64_t group_h, int64_t group_i,
                       const uint32_t* table, float limit, int h_bf16, float* out, int threads);
void oracle_nearest(const float* v, int64_t n, const float* w, int64_t w_stride, const float* grid, int64_t G,
                    int64_t* out);
int oracle_max_threads(void);

static uint32_t rng = 12345u;
static uint32_t next(void) { rng = rng * 1664525u + 1013904223u; return rng; }
static float unit(void) { return (float)(next() >> 8) / 16777216.0f - 0.5f; }
#define ARR(type, name, n) type* name = (type*)malloc(sizeof(type) * (size_t)(n) + 1)

int main(void) {
  uint32_t table[256], table8[256];
  for (int i = 0; i < 256; ++i) table[i] = next(), table8[i] = next();
  enum { E = 3, H = 64, I = 32, T = 2, K = 2, NH = 2 };
  ARR(uint16_t, codes, 7); for (int i = 0; i < 7; ++i) codes[i] = (uint16_t)next();
  ARR(float, dec, 7 * 8);
  oracle_e8p_decode(codes, 0, table, dec);
  oracle_e8p_decode(codes, 7, table, dec);
  /* projections: gate/up [E, I, H/8], down [E, H, I/8]; group 32 for H, 16 for I */
  ARR(uint16_t, gc, E * I * H / 8); ARR(uint16_t, uc, E * I * H / 8); ARR(uint16_t, dc, E * H * I / 8);
  ARR(float, gs, E * I * (H / 32)); ARR(float, us, E * I * (H / 32)); ARR(float, ds, E * H * (I / 16));
  for (int i = 0; i < E * I * H / 8; ++i) gc[i] = (uint16_t)next(), uc[i] = (uint16_t)next();
  for (int i = 0; i < E * H * I / 8; ++i) dc[i] = (uint16_t)next();
  for (int i = 0; i < E * I * (H / 32); ++i) gs[i] = 0.01f * (1 + (next() & 7)), us[i] = gs[i];
  for (int i = 0; i < E * H * (I / 16); ++i) ds[i] = 0.01f * (1 + (next() & 7));
  ARR(float, x, T * H); for (int i = 0; i < T * H; ++i) x[i] = unit() * 8.f;
  int32_t idx[T * K] = {0, 2, 1, 2}, lhs[T * K] = {1, 0, 1, 0}, hot[E] = {-1, 1, 0};
  float w[T * K] = {0.75f, 0.25f, 0.5f, 0.5f};
  ARR(float, y, T * K * I);
  oracle_routed_matvec(x, gc, gs, table, idx, NULL, T * K, K, I, H, 32, y, 2);
  oracle_routed_matvec(x, gc, gs, table, idx, lhs, T * K, 1, I, H, 32, y, 2);
  oracle_routed_matvec(x, gc, gs, table, idx, NULL, 0, K, I, H, 32, y, 2);
  ARR(uint8_t, rgc, NH * I * H / 8); ARR(uint8_t, ruc, NH * I * H / 8); ARR(uint8_t, rdc, NH * H * I / 8);
  ARR(float, rgs, NH * I * (H / 64)); ARR(float, rus, NH * I * (H / 64)); ARR(float, rds, NH * H * (I / 32));
  for (int i = 0; i < NH * I * H / 8; ++i) rgc[i] = (uint8_t)next(), ruc[i] = (uint8_t)next();
  for (int i = 0; i < NH * H * I / 8; ++i) rdc[i] = (uint8_t)next();
  for (int i = 0; i < NH * I * (H / 64); ++i) rgs[i] = 0.001f, rus[i] = 0.002f;
  for (int i = 0; i < NH * H * (I / 32); ++i) rds[i] = 0.003f;
  int32_t rrows[T * K] = {-1, 1, 0, -1};
  oracle_routed_matvec8(x, rgc, rgs, table8, rrows, NULL, T * K, K, I, H, 64, y, 2);
  ARR(float, out, T * H);
  oracle_moe_decode(x, T, H, I, idx, w, K, gc, gs, uc, us, dc, ds, 32, 16, table, 0.f, 1, out, 2);
  oracle_moe_decode(x, T, H, I, idx, w, K, gc, gs, uc, us, dc, ds, 32, 16, table, 7.f, 0, out, 1);
  oracle_moe_decode(x, 0, H, I, idx, w, K, gc, gs, uc, us, dc, ds, 32, 16, table, 0.f, 1, out, 2);
  oracle_moe_decode_nested(x, T, H, I, idx, w, K, gc, gs, uc, us, dc, ds, 32, 16, table, 0.f, 1, hot, rgc, rgs, ruc,
                           rus, rdc, rds, 64, 32, table8, out, 2);
  /* non-finite h through the bf16 rounding */
  x[0] = INFINITY; x[1] = NAN; x[H] = 3.0e38f;
  oracle_moe_decode(x, T, H, I, idx, w, K, gc, gs, uc, us, dc, ds, 32, 16, table, 0.f, 1, out, 2);
  /* nearest: unweighted, one shared weight vector, one per vector, empty */
  ARR(float, grid, 256 * 8); for (int i = 0; i < 256 * 8; ++i) grid[i] = unit() * 4.f;
  ARR(float, v, 5 * 8); for (int i = 0; i < 5 * 8; ++i) v[i] = unit() * 4.f;
  ARR(float, wv, 5 * 8); for (int i = 0; i < 5 * 8; ++i) wv[i] = 0.5f + unit();
  int64_t near[5];
  oracle_nearest(v, 5, NULL, 0, grid, 256, near);
  oracle_nearest(v, 5, wv, 0, grid, 256, near);
  oracle_nearest(v, 5, wv, 8, grid, 256, near);
  oracle_nearest(v, 0, wv, 8, grid, 256, near);
  for (int i = 0; i < 5; ++i)
    if (near[i] < 0 || near[i] >= 256) return 2;
  if (oracle_max_threads() < 1) return 3;
  free(codes); free(dec); free(gc); free(uc); free(dc); free(gs); free(us); free(ds); free(x); free(y);
  free(rgc); free(ruc); free(rdc); free(rgs); free(rus); free(rds); free(out); free(grid); free(v); free(wv);
  printf("ok\n");
  return 0;
}
